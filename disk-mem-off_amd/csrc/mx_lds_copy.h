// Global -> LDS copies by the buffer loads' LDS mode, and the wait that ends a ring stage.
#pragma once

#include <hip/hip_runtime.h>

typedef __attribute__((address_space(3))) void mx_lds_void;

// One 16-byte piece per lane from global memory into LDS: lane l's piece lands at
// dst + 16 l.  aux: cache-policy bits of the load.
template <int AUX = 0>
__device__ __forceinline__ void mx_copy_to_lds16(__amdgpu_buffer_rsrc_t r, char* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (mx_lds_void*)dst, 16, off, 0, 0, AUX);
}

// Wait until at most N vector memory operations of this wave are outstanding, then meet
// the other waves at a barrier.  No memory fence on the way in (a release fence on LDS
// would wait for every copy into LDS still in flight); the acquire fence after the
// barrier keeps the compiler from moving the next LDS reads above it.
template <int N>
__device__ __forceinline__ void mx_wait_copies_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
