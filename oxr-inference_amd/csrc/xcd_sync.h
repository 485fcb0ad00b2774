// Cooperation among the workgroups of one XCD inside a launch (gfx950, MI355X single partition).
//
// A launch of kGrid = 256 workgroups, each sized to own a whole CU (LDS above half a CU's), puts 32
// on each of the 8 XCDs.  A workgroup reads its XCD from the hardware (HW_REG_XCC_ID) and takes
// rank blockIdx.x / 8 among the XCD's workgroups, the dispatcher placing workgroups on XCDs
// round-robin; each sets its rank's bit in its XCD's census word, so a placement that breaks this is
// reported in the error word.  Workgroups of one XCD hand data to each other through the XCD's L2:
// plain stores, a wait for their completion, an atomic add on an XCD counter; the waiters poll the
// counter with sc1 loads and read the data with sc0 loads (L1 bypassed) -- measured exact on
// MI355X, where an sc0 poll could return a stale counter after an atomic to another line.  Every
// wait is bounded: one that cannot complete sets a bit of the error word and goes on, so a launch
// always ends.
//
// Control words (uint32) at the start of a kernel's workspace: one 256-byte block per XCD (census,
// two phase counters, finished count) and then the error word.  The last workgroup of an XCD to
// finish zeroes that XCD's block (every other one has passed its last wait by then), so a launch
// leaves its control words as it found them: zero before the first launch, zero after each.
#pragma once

#include "common.h"

namespace oxr {
namespace xcd {

constexpr int kXcds = 8;
constexpr int kXcdWgs = 32;
constexpr int kGrid = kXcds * kXcdWgs;
constexpr uint32_t kSpinLimit = 1u << 16;
constexpr int kCtlStride = 64;  // uint32 words per XCD block
enum Ctl { kCensus = 0, kPhase0 = 1, kPhase1 = 2, kExit = 3 };
constexpr int kErrorWord = kXcds * kCtlStride;
constexpr size_t kCtlBytes = 4096;
enum Error : uint32_t { kErrPlacement = 1, kErrPhase0Wait = 2, kErrPhase1Wait = 4 };

__device__ __forceinline__ uint32_t xcc_id() {
  uint32_t v;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
  return v & 0xfu;
}

__device__ __forceinline__ uint32_t load_sc1(const uint32_t* p) {
  const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)p, 0, 4, 0x00020000);
  return __builtin_amdgcn_raw_buffer_load_b32(r, 0, 0, 16);
}

__device__ __forceinline__ uint32_t atomic_add(uint32_t* p, uint32_t v) {
  return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void set_error(uint32_t* ctl_base, uint32_t bits) {
  __hip_atomic_fetch_or(ctl_base + kErrorWord, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Until *ctr >= target (one wave, all lanes); false after kSpinLimit polls.
__device__ __forceinline__ bool wait_count(const uint32_t* ctr, uint32_t target) {
  for (uint32_t n = 0; n < kSpinLimit; ++n) {
    if (__builtin_amdgcn_readfirstlane(load_sc1(ctr)) >= target) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// Every memory operation this wave has issued has completed (stores are in L2) before what follows.
__device__ __forceinline__ void stores_done() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0);
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Count this workgroup into an XCD counter (lane 0), then wait until the atomic has been performed
// (an atomic without return still holds the vector memory counter until it is acknowledged).
__device__ __forceinline__ void arrive(uint32_t* ctr, int lane) {
  if (lane == 0) atomic_add(ctr, 1u);
  stores_done();
}

// The workgroup barrier alone: no memory fence, so no wave waits for its loads in flight.
__device__ __forceinline__ void barrier() { asm volatile("s_barrier" ::: "memory"); }

// 1 KiB blocks of a packed buffer into LDS, L1 bypassed (sc0): block j of `src` to dst + 512 j
// elements; lane i of a block writes its bytes [16 i, 16 i + 16).
__device__ __forceinline__ void copy_block_to_lds(const bf16_t* src, bf16_t* dst, int lane) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(src + lane * 8),
                                   (void __attribute__((address_space(3)))*)dst, 16, 0, 1);
}
__device__ __forceinline__ void copy_to_lds(const bf16_t* src, bf16_t* dst, int n, int lane) {
  for (int j = 0; j < n; ++j) copy_block_to_lds(src + j * 512, dst + j * 512, lane);
}

// Census (lane 0 of one wave per workgroup): flags a rank seen twice on an XCD, or an XCD past 8.
__device__ __forceinline__ void census(uint32_t* ctl_base, uint32_t* ctl, int rank, uint32_t xcc, int lane) {
  if (lane == 0) {
    const uint32_t seen = __hip_atomic_fetch_or(ctl + kCensus, 1u << rank, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (((seen >> rank) & 1u) || xcc >= (uint32_t)kXcds) set_error(ctl_base, kErrPlacement);
  }
}

// The workgroup's last use of the control words (one wave, after its last wait): the XCD's last
// workgroup zeroes the block.
__device__ __forceinline__ void finish(uint32_t* ctl, int lane) {
  if (lane == 0 && atomic_add(ctl + kExit, 1u) == (uint32_t)(kXcdWgs - 1)) {
    ctl[kCensus] = 0u;
    ctl[kPhase0] = 0u;
    ctl[kPhase1] = 0u;
    ctl[kExit] = 0u;
  }
}

// Host: the device is an MI355X in its single-partition mode (one workgroup per CU on 256 CUs).
inline bool device_fits() {
  static int cached = -1;
  if (cached < 0) {
    int dev = 0, cus = 0;
    cached = hipGetDevice(&dev) == hipSuccess &&
                     hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
                     cus == kGrid
                 ? 1
                 : 0;
  }
  return cached == 1;
}

}  // namespace xcd
}  // namespace oxr
