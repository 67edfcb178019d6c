// Grid-wide arrival counting for persistent kernels (every workgroup resident).
//
// A workgroup signals once per call with an atomic add on one of up to 32
// sub-counters (workgroup b counts in b % NSUB), so no address takes more than
// ceil(G / 32) serialised atomics; waiters poll the 32 words with one wave-wide
// load.  Counters are never reset:
// call number n (the generation, kept in the same block) waits for sub-counter s to
// reach n * (workgroups counted in s), modulo 2^32.
//
// Memory: data published before an arrival must be written with agent-scope
// stores (written through to the level all XCDs share) and be complete
// (s_waitcnt vmcnt(0) in the publishing wave) before the arrival; readers use
// agent-scope loads after the wait.  Polls give up after SPIN_LIMIT sleeps and
// count a timeout, so every wave always exits.
#pragma once

#include "common.h"

namespace cachalot {
namespace gsync {

constexpr int NSUB_MAX = 32;
constexpr int LINE = 128;                       // one counter per cache line
constexpr int OFF_GEN = 0;                      // u32 generation
constexpr int OFF_TIMEOUTS = 4;                 // u32 waits that gave up
constexpr int OFF_SUB = LINE;
constexpr int BYTES = OFF_SUB + NSUB_MAX * LINE;   // one barrier block
constexpr unsigned int SPIN_LIMIT = 1u << 22;

__device__ __forceinline__ uint32_t* word(uint8_t* blk, int off) { return reinterpret_cast<uint32_t*>(blk + off); }

__device__ __forceinline__ uint32_t load_agent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Generation of this call (read once at kernel start by every workgroup).
__device__ __forceinline__ uint32_t next_generation(uint8_t* gen_blk) { return load_agent(word(gen_blk, OFF_GEN)) + 1u; }

__host__ __device__ inline int nsub(int G) { return G < NSUB_MAX ? G : NSUB_MAX; }

// One lane per workgroup: count this workgroup in sub-counter b % NSUB.  The add's
// result is consumed, so it is performed where every XCD sees it before the wave
// goes on (a non-returning add was observed to become visible ~2 us later).
__device__ __forceinline__ void arrive(uint8_t* bar) {
  const int s = (int)blockIdx.x % nsub((int)gridDim.x);
  uint32_t old = __hip_atomic_fetch_add(word(bar, OFF_SUB + s * LINE), 1u, __ATOMIC_RELAXED,
                                        __HIP_MEMORY_SCOPE_AGENT);
  asm volatile("" ::"v"(old));
}

// A whole wave: wait until every workgroup of generation `gen` has arrived (each
// sub-counter s at gen * (workgroups counted in s), lane s polling it).  Returns
// false on timeout.  The kernel records the generation with finish() once, in one
// workgroup, after this wait (so after every workgroup has read the old value).
__device__ __forceinline__ bool wait(uint8_t* bar, uint8_t* gen_blk, uint32_t gen, int lane) {
  const int G = (int)gridDim.x, ns = nsub(G);
  const uint32_t per = (uint32_t)((G - lane + ns - 1) / ns);
  const uint32_t* sub = word(bar, OFF_SUB + (lane < ns ? lane : 0) * LINE);
  const uint32_t target = gen * per;
  bool ok = true;
  for (unsigned int polls = 0;; ++polls) {
    const bool done = lane >= ns || (int)(load_agent(sub) - target) >= 0;
    if (__all(done)) break;
    if (polls >= SPIN_LIMIT) {
      if (lane == 0) atomicAdd(word(gen_blk, OFF_TIMEOUTS), 1u);
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return ok;
}

// Record the generation of a finished call (one lane of one workgroup, after wait()).
__device__ __forceinline__ void finish(uint8_t* gen_blk, uint32_t gen) {
  __hip_atomic_store(word(gen_blk, OFF_GEN), gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Agent-scope (write-through) stores for data other workgroups read after a barrier.
__device__ __forceinline__ void store_agent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace gsync
}  // namespace cachalot
