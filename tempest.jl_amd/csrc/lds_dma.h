// Device helpers shared by the product and attention kernels: direct global
// -> LDS loads on gfx950 and a compile-time loop.
//
// buffer_load_dwordx4 ... lds writes each lane's 16 bytes at M0 + 16 lane, so
// one wave instruction fills 1 KB of LDS with no staging registers.  It is
// issued from inline assembly: the compiler, seeing an LDS write by DMA,
// would otherwise make later LDS reads (ds_read_b64_tr_b16 among them) wait
// for every outstanding global load, serializing a pipelined sweep.  The
// caller waits for completion explicitly (wait_and_meet) before the stage it
// fills is read.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <utility>

namespace th_dev {

template <int... I, typename F>
__device__ __forceinline__ void static_for_impl(std::integer_sequence<int, I...>, F&& f) {
  (f(std::integral_constant<int, I>{}), ...);
}
// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>), unrolled.
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(std::make_integer_sequence<int, N>{}, f);
}

// One 16-byte lane load from global memory (buffer `rsrc`, byte offset
// voff + soff) straight into LDS at byte m0 + 16 lane.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, int32_t voff, int32_t soff, uint32_t m0) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(m0));
}

// The same for a stream read once: non-temporal, so that it does not evict
// from L2 what other loads reuse.
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t rsrc, int32_t voff, int32_t soff, uint32_t m0) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen nt lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(m0));
}

// One 4-byte lane load from global memory straight into LDS at byte
// m0 + 4 lane.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rsrc, int32_t voff, int32_t soff, uint32_t m0) {
  asm volatile("buffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(rsrc), "s"(soff), "{m0}"(m0));
}

// Wait until this wave has at most N vector memory operations in flight and
// no LDS reads, then meet the other waves of the workgroup.
template <int N>
__device__ __forceinline__ void wait_and_meet() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"i"(N) : "memory");
}

// A buffer resource over [base, base + 2 GiB): loads past the array are the
// caller's to avoid (the builders check that every sweep stays inside).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_of(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}

}  // namespace th_dev
