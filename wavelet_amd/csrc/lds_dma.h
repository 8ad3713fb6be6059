// LDS-DMA helpers for gfx950: HBM -> LDS copies without register staging
// (global_load_lds_dwordx4: lane i of a wave instruction lands at the LDS
// address in M0 + 16 i), the waits for them, and an LDS barrier.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace wkv {

// The copies, the waits for them and the barriers are written as inline asm
// so the compiler's own wait-count insertion never sees an LDS write it would
// have to wait for: it cannot always prove that a read of one step buffer
// does not alias the copies still landing in the others, and then waits for
// every outstanding copy (vmcnt(0)), which would drain the pipeline. The
// "memory" clobbers keep the compiler from moving LDS accesses across them.
// M0 carries the LDS address of an LDS-DMA copy; nothing else in the kernel
// uses M0, and each copy sets it immediately before use.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void copy16_to_lds(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
// The same copy through a buffer resource: 16 bytes at voff + soff of the
// resource's base (voff per lane, soff uniform: one SGPR offset per copy
// instead of a 64-bit address add per lane).
__device__ __forceinline__ void buffer_copy16_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                                     uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(lds), "v"(voff), "s"(r),
               "s"(soff)
               : "memory", "m0");
}
// NCP copies of 1 KB under one M0 write: copy k lands at lds + 1024 k. The
// LDS address of a copy is M0 + its instruction offset + 16 x lane, and the
// instruction offset (1024 k here) is added to the memory address as well, so
// the SGPR offset of copy k is k x sdelta with sdelta = (source stride of the
// copies) - 1024. One M0 write per run instead of one per copy.
template <int NCP>
__device__ __forceinline__ void buffer_copy16_run_to_lds(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t sdelta,
                                                         uint32_t lds) {
  static_assert(NCP >= 1 && NCP <= 4, "instruction offsets below 4096");
  if constexpr (NCP == 1) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(lds), "v"(voff),
                 "s"(r)
                 : "memory", "m0");
  } else if constexpr (NCP == 2) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
                 "buffer_load_dwordx4 %1, %2, %3 offen offset:1024 lds" ::"s"(lds),
                 "v"(voff), "s"(r), "s"(sdelta)
                 : "memory", "m0");
  } else {
    const uint32_t s2 = 2 * sdelta, s3 = 3 * sdelta;
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
                 "buffer_load_dwordx4 %1, %2, %3 offen offset:1024 lds\n\t"
                 "buffer_load_dwordx4 %1, %2, %4 offen offset:2048 lds\n\t"
                 "buffer_load_dwordx4 %1, %2, %5 offen offset:3072 lds" ::"s"(lds),
                 "v"(voff), "s"(r), "s"(sdelta), "s"(s2), "s"(s3)
                 : "memory", "m0");
  }
}
#pragma clang diagnostic pop

// Waits until at most N of this wave's vector-memory operations are pending.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// p[min(idx, n - 1)] for idx < n, else -1 (n >= 1), loaded and waited for in
// one asm block: the compiler's wait-count insertion never sees a load whose
// result it would guard with a vmcnt(0) at every later use, a wait that would
// also drain the LDS-DMA copies in flight. The wait here drains them too, so
// a kernel calls this rarely.
__device__ __forceinline__ int load_i32_drained(const int32_t *p, int idx, int n) {
  const int32_t *a = p + (idx < n ? idx : n - 1);
  int v;
  asm volatile("global_load_dword %0, %1, off\n\ts_waitcnt vmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return idx < n ? v : -1;
}

// Workgroup barrier for LDS: this wave's LDS accesses complete, then s_barrier.
__device__ __forceinline__ void barrier_lds() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void *)p));
}

}  // namespace wkv
