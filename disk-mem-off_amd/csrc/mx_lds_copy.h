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

// Chunk rotation of the 1 KiB operand fragments (16 rows x 64 bytes) that the LDS copies
// fill and the MFMA operand reads consume: row j's 16-byte chunk c sits at slot
// 4 j + (c + mx_frag_rot(j)) mod 4.  The rotation keeps the four chunks of a row in its own
// 64 bytes (so four consecutive copy lanes still read one row's 64 contiguous bytes).  With
// rotation (j / 2) mod 4 the 16-byte reads of lanes (j, c) = (lane % 16, lane / 16) run
// without bank-conflict cycles on gfx950 (SQ_LDS_BANK_CONFLICT 0, as for 64 lanes reading 1
// KiB in order); the rotations (j / 4 + 2 ((j / 2) mod 2)) mod 4, (j / 4) mod 4, j mod 4 and
// none each double the LDS cycles of the read (measured with a read-only probe).
__device__ __forceinline__ int mx_frag_rot(int j) { return (j >> 1) & 3; }
// Copy lane l's chunk (it loads row l / 4) and the byte offset of lane (j, c)'s operand.
__device__ __forceinline__ int mx_frag_copy_chunk(int l) { return ((l & 3) - mx_frag_rot(l >> 2)) & 3; }
__device__ __forceinline__ int mx_frag_read_pos(int j, int c) {
  return (4 * j + ((c + mx_frag_rot(j)) & 3)) * 16;
}
