// Direct HBM -> LDS tile staging for the attention kernels (gfx950).
//
// global_load_lds_dwordx4 moves 16 bytes per lane from global memory straight
// into LDS: lane L of one instruction writes LDS bytes [M0 + 16 L, M0 + 16 L + 16),
// so one wave-instruction fills 1 KB of LDS.  No VGPR staging and no ds_write
// are needed, and the copy of the next tile runs while the current one is
// being multiplied.
//
// The loads are issued from inline assembly and completed with an explicit
// "s_waitcnt vmcnt(0)" before the workgroup barrier that publishes a stage.
// (Through the compiler builtin, every LDS read after any LDS-DMA gets a
// vmcnt(0) in front of it, which would serialise the prefetch with the math.)
// The compiler does not count these loads; its own vmcnt waits for other loads
// stay correct because loads retire in issue order (a wait for an older load
// can only become stricter).  The asm statements carry no "memory" clobber:
// ordering against the LDS reads of a stage comes from the workgroup barrier
// (a fence) between them, and without the clobber the compiler keeps the
// read-only list and mask loads on the scalar unit instead of turning them
// into vector loads whose waits would also drain the in-flight tile copy.
// Loads whose results a loop consumes must be completed before the loop
// (consume_regs), or the compiler's first-use wait inside the loop would
// drain the tile copy on every iteration.
//
// LDS tiles are padded by 16 bytes per row, which keeps the MFMA operand reads
// (ds_read_b128 of 32 consecutive rows at one column) free of bank conflicts.
// A padded tile of R rows x W bytes occupies R * (W + 16) bytes, a whole
// number of KB for the tiles used here; lanes whose 16-byte LDS slot is a
// row's padding re-read the first chunk of that row (harmless, L2-resident).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __attribute__((address_space(3))) void prism_lds_void;

// 32-bit LDS address of a __shared__ object
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(prism_lds_void*)(p); }

__device__ __forceinline__ uint32_t uniform_u32(uint32_t x) { return __builtin_amdgcn_readfirstlane(x); }
// (readfirstlane returns int: each half goes through uint32_t so the low word
// is zero-extended, not sign-extended, into the 64-bit address)
__device__ __forceinline__ const void* uniform_ptr(const void* p) {
  const uint64_t u = (uint64_t)(uintptr_t)p;
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)u);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(u >> 32));
  return (const void*)(uintptr_t)(lo | (hi << 32));
}

// 16 bytes per lane: LDS[m0 + 16*lane] <- global[base + voff]
__device__ __forceinline__ void dma_b128(uint32_t voff, const void* base, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(m0) : "m0");
}
// 4 bytes per lane: LDS[m0 + 4*lane] <- global[base + voff]
__device__ __forceinline__ void dma_b32(uint32_t voff, const void* base, uint32_t m0) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(m0) : "m0");
}
// wait until every load this wave issued (DMA included) has landed
__device__ __forceinline__ void dma_wait_all() { asm volatile("s_waitcnt vmcnt(0)"); }

// Scalar loads of wave-uniform, read-only data (list entries, validity
// words), completed inside the asm.  They use lgkmcnt, so they never wait for
// the in-flight tile copy (a compiler-generated vector load of the same data
// would be followed by a vmcnt(0)).
__device__ __forceinline__ int sload_i32(const int32_t* p) {
  int v;
  asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(uniform_ptr(p)));
  return v;
}
__device__ __forceinline__ uint64_t sload_u64(const uint64_t* p) {
  uint64_t v;
  asm volatile("s_load_dwordx2 %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(uniform_ptr(p)));
  return v;
}

// Make the compiler complete the loads that produced x here (it inserts the
// s_waitcnt before an asm statement that reads the registers).
template <typename T>
__device__ __forceinline__ void consume_regs(const T& x) {
  asm volatile("" ::"v"(x));
}

// Byte offset, inside a row-major global tile of rows of W bytes, that lane
// `lane` of KB-instruction `i` fetches for a padded LDS tile (pitch W + 16).
template <int W>
__device__ __forceinline__ uint32_t padded_src_offset(int i, int lane) {
  constexpr int P = W + 16;
  const int pos = 1024 * i + 16 * lane;
  const int row = pos / P, col = pos - row * P;
  return (uint32_t)(row * W + (col < W ? col : 0));
}
