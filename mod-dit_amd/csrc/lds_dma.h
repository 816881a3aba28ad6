// Direct global -> LDS staging helpers shared by the attention kernels (gfx950).
#pragma once

#include "common.h"

namespace moddit {

// buffer_load_dwordx4 ... lds: lane l writes its 16 bytes at LDS byte m0 + 16*l. Issued as
// inline asm so the compiler does not track it: it would otherwise wait for every
// outstanding DMA before each LDS read it cannot disambiguate. Completion is established
// explicitly (s_waitcnt vmcnt(0) + barrier) before any wave reads the written stage;
// vmcnt waits the compiler emits for its own loads stay correct because vector loads
// retire in issue order.
// The hazard recognizer does not look inside inline asm, so the asm supplies the wait
// states itself: an LDS DMA must not issue in the cycle after an SALU write of m0 (the
// compiler writes m0 right before the asm), and a VMEM instruction needs 5 wait states
// after a VALU write (v_readlane / v_readfirstlane, e.g. a spilled descriptor being
// reloaded) of an SGPR it reads. Without them the load can pick up the previous m0 or a
// stale descriptor word and land in, or come from, the wrong place.
static __device__ __forceinline__ void lds_dma16(u32x4 rsrc, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
               :
               : "v"(voff), "s"(rsrc), "s"(soff), "{m0}"(lds)
               : "memory");
}

// Raw buffer descriptor: base, stride 0, num_records = bytes (range checked per lane).
static __device__ __forceinline__ u32x4 raw_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return u32x4{static_cast<uint32_t>(a), static_cast<uint32_t>(a >> 32) & 0xffffu, bytes,
               0x00020000u};
}

static __device__ __forceinline__ uint32_t lds_addr(const unsigned char* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
      (__attribute__((address_space(3))) const unsigned char*)(p)));
}

}  // namespace moddit

// s_waitcnt with lgkmcnt(0) and vmcnt(n), n < 16 (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8]); expcnt is left unconstrained. Used to retire all but the n most recent
// DMA stages before the barrier that publishes a ring stage.
#define MODDIT_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(0x0070 | (n))
