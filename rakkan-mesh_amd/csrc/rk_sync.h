// rk_sync.h — hand-offs between the workgroups of one launch, for gfx950:
// counts and flags (the values-and-Wo launch) and tagged words (the
// one-token MoE feed-forward).
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

// A tagged word carries 48 bits of data under a 16-bit tag: the low bits of
// the launch's number. Every workgroup learns that number from count words
// of its own: each counts the launches that covered a fixed part of the
// work, and is read and written only by the workgroup covering that part,
// so (launches of a stream running in order) every count holds the same
// number during a launch, whatever the launch's grid. A writer stores its
// words with agent-scope stores (written through to where every XCD's loads
// of that scope look) and goes on; a reader polls them with agent-scope
// loads until each carries its launch's tag. No word is ever reset, no
// store waits for another, and there is no atomic (adds to one address
// serialise, tens of ns each on MI355X, and a store's acknowledgement takes
// about a microsecond). Measured: in the one-token MoE launch (192 and 256
// workgroups on either side of its last hand-off) tagged words beat counts
// and flags by several microseconds; in the values-and-Wo launch (128 and
// 128) counts and flags stay faster (13.4 against 15.3 us a layer at the
// 8B shape), so that launch keeps them. Every poll is bounded by the device's real-time clock (kSyncTimeout); a
// reader that gives up sets an error word, which the owner reports after
// the step, and goes on with what memory holds.

// The launch's number for a workgroup covering the parts of count words
// cnt[0..n): one more than the first (c0, loaded by every thread as early as
// possible: the load's wait falls at the number's first use), written back
// to all of them by thread 0.
__device__ __forceinline__ unsigned long long tag_take(unsigned long long c0, unsigned long long *cnt, int n) {
    const unsigned long long v = c0 + 1;
    if (threadIdx.x == 0)
        for (int i = 0; i < n; i++) cnt[i] = v;
    return v;
}

__device__ __forceinline__ uint32_t tag_of(unsigned long long n) { return (uint32_t)n & 0xFFFFu; }

// A Q8_0 block (32 codes, then the scale: 36 bytes) as six tagged words of
// six bytes each: a reader holding the six words of its launch holds the
// block. By one wave (every lane calls it): lanes 0-7 hold four codes each
// (pk) and the scale d.
__device__ __forceinline__ void tag_put_q8(unsigned long long *w, uint32_t pk, float d, uint32_t tag) {
    const int lane = threadIdx.x & 63;
    const int i = min(lane, 5), j0 = (6 * i) >> 2, o = (6 * i) & 3;  // bytes 6i.. from dword j0, byte o (0 or 2)
    const uint32_t lo = __shfl(pk, j0), hi0 = __shfl(pk, min(j0 + 1, 7));
    const uint32_t hi = j0 + 1 == 8 ? f2u(d) : hi0;  // (lane 5: its own scale)
    const unsigned long long bytes = (((unsigned long long)hi << 32) | lo) >> (8 * o);
    if (lane < 6)
        __hip_atomic_store(w + lane, ((unsigned long long)tag << 48) | (bytes & 0xFFFFFFFFFFFFull), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}

// Block b's words in `want` (bit i: word i) that carry the tag, read into
// LDS (codes sq [block][32], scale ss [block]); returns the bits read.
__device__ __forceinline__ int tag_q8_words(const unsigned long long *w, int b, int want, uint32_t tag, int8_t *sq,
                                            float *ss) {
    int got = 0;
#pragma unroll
    for (int i = 0; i < 6; i++) {
        if (!(want >> i & 1)) continue;
        const unsigned long long v = __hip_atomic_load(w + 6 * b + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((uint32_t)(v >> 48) != tag) continue;
        got |= 1 << i;
        if (i == 5) {
            *reinterpret_cast<uint16_t *>(sq + 32 * b + 30) = (uint16_t)v;
            ss[b] = u2f((uint32_t)(v >> 16));
        } else {
            uint16_t *dst = reinterpret_cast<uint16_t *>(sq + 32 * b + 6 * i);
            dst[0] = (uint16_t)v;
            dst[1] = (uint16_t)(v >> 16);
            dst[2] = (uint16_t)(v >> 32);
        }
    }
    return got;
}

// The nblk (<= 4·NT) tagged Q8_0 blocks of w into LDS, by a workgroup of NT
// threads (thread t takes blocks t, t + NT, ...). While fewer than half of
// the blocks are in, a round reads only a block's last word (two codes and
// the scale: one word a block of polling); a block whose last word is in
// reads the other five in the next round; from half on, a round reads all
// of a missing block's words (one round trip after its stores land). Ends
// with a barrier. s_to: a word of static LDS.
template <int NT>
__device__ void tag_get_q8(const unsigned long long *w, int nblk, uint32_t tag, int8_t *sq, float *ss,
                           unsigned long long *err, int *s_to) {
    const int tid = threadIdx.x;
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    if (tid == 0) *s_to = 0;
    int have[4];  // words in, per block of this thread (63: all, or no block)
#pragma unroll
    for (int j = 0; j < 4; j++) have[j] = tid + NT * j < nblk ? 0 : 63;
    bool full = false;
    for (int it = 0; it < (1 << 24); it++) {
        bool mine = true;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (have[j] != 63)
                have[j] |= tag_q8_words(w, tid + NT * j, full || (have[j] & 32) ? 63 & ~have[j] : 32, tag, sq, ss);
            mine = mine && have[j] == 63;
        }
        if (tid == 0 && __builtin_amdgcn_s_memrealtime() - t0 > kSyncTimeout) *s_to = 1;
        if (__syncthreads_count(mine) == NT || *s_to) break;
        full = full || 2 * __syncthreads_count(tid < nblk && (have[0] & 32)) >= min(nblk, NT);
        __builtin_amdgcn_s_sleep(1);
    }
    if (tid == 0 && *s_to) __hip_atomic_store(err, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
}

}  // namespace rk
