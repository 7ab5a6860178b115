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
// The LDS layout of the tiles (quads of rows, chunks swizzled) is described with
// RowTile below; each tile is a whole number of KB, so a stage is filled by a
// fixed number of KB-instructions spread over the waves.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mfma.h"

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
// 4 bytes per lane: LDS[m0 + 4*lane] <- global[base + 4*lane]; the lane
// offset is formed inside the asm, so no register holds it between copies
__device__ __forceinline__ void dma_b32_rows(const void* base, uint32_t m0) {
  uint32_t t;
  asm volatile(
      "v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0\n\tv_lshlrev_b32 %0, 2, %0\n\t"
      "s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1"
      : "=&v"(t)
      : "s"(base), "s"(m0)
      : "m0");
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

template <int N>
__device__ __forceinline__ void dma_wait_le() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N));
}

// ------------------------------------------------------------ stage pipeline
// The attention kernels walk a list of entries (prism_pair_union) with an
// NST-stage ring of LDS stages: the tiles of entry j + NST - 1 are copied while
// entry j is multiplied.  At the top of iteration j the copies of entries
// j+1 .. min(j+NST-2, n-1) may stay in flight; CNT = copy instructions per
// entry issued by this wave.
template <int NST, int CNT>
__device__ __forceinline__ void stage_wait(int after) {  // after = n - 1 - j
  static_assert(NST >= 2 && NST <= 4, "2 to 4 stages");
  if constexpr (NST >= 4) {
    if (after >= 2) {
      dma_wait_le<2 * CNT>();
      return;
    }
  }
  if constexpr (NST >= 3) {
    if (after >= 1) {
      dma_wait_le<CNT>();
      return;
    }
  }
  dma_wait_le<0>();
}

// Wave-uniform ring of the next NST list entries, read with scalar loads.
// (A vector load of the list would put a vmcnt wait in the loop: the
// compiler cannot tell which iteration issued it, so it waits for every load
// in flight at the loop latch, tile copies included.)  The scalar loads wait
// on lgkmcnt, which at the top of an iteration only covers the LDS reads of
// the previous entry, all consumed by then; consecutive entries share a
// scalar cache line.
template <int NST>
struct EntryRing {
  int e[NST];  // entries j .. j + NST - 1 (0 past the end of the list)
  __device__ __forceinline__ void init(const int32_t* U, int n) {
#pragma unroll
    for (int k = 0; k < NST; ++k) e[k] = k < n ? sload_i32(U + k) : 0;
  }
  // shift the ring from entry j to j + 1
  __device__ __forceinline__ void advance(const int32_t* U, int n, int j) {
#pragma unroll
    for (int k = 0; k + 1 < NST; ++k) e[k] = e[k + 1];
    const int k = j + NST;
    e[NST - 1] = k < n ? sload_i32(U + k) : 0;
  }
};
// stage holding entry j + NST - 1 when entry j is in stage st
template <int NST>
__device__ __forceinline__ int stage_ahead(int st) {
  return st == 0 ? NST - 1 : st - 1;
}

// ------------------------------------------------------------ work queue
// Persistent launches (queue != null): the queue holds kQueueLanes counters,
// one per XCD.  Launch position b belongs to lane b mod 8: the XCD to which
// the hardware's round-robin dispatch sends workgroup b of a launch with one
// workgroup per pair, so each XCD walks the same runs of neighbouring pairs
// as there (their lists overlap in its L2).  A workgroup starts on the lane of
// its own XCD (blockIdx mod 8) and takes b = 8 atomicAdd(counter, 1) + lane;
// when its lane runs out it moves to the next lane, taking the remaining work
// of a slower XCD, until all eight are exhausted.  Each position is taken
// exactly once whichever XCD a workgroup runs on.  The position is published
// through LDS between two barriers (the first also keeps the next pair's tile
// copies off the LDS that slower waves still read), so all waves of the
// workgroup take the same positions and leave the loop together.
constexpr int kQueueLanes = 8;

// the queue state of a workgroup, in LDS (so no register stays live across
// the pairs): the published position, the current lane and the number of
// lanes not yet found exhausted (both used by thread 0 only)
struct WorkQueueState {
  int slot, lane, left;
};

__device__ __forceinline__ void work_queue_init(WorkQueueState* st) {
  if (threadIdx.x == 0) {
    st->lane = (int)(blockIdx.x % kQueueLanes);
    st->left = kQueueLanes;
  }
}

// next launch position, or -1 when every lane is exhausted
__device__ __forceinline__ int work_queue_take(int* queue, int total, WorkQueueState* st) {
  __syncthreads();
  if (threadIdx.x == 0) {
    int r = -1;
    while (st->left > 0) {
      const int b = kQueueLanes * atomicAdd(queue + st->lane, 1) + st->lane;
      if (b < total) {
        r = b;
        break;
      }
      st->lane = (st->lane + 1) % kQueueLanes;
      --st->left;
    }
    st->slot = r;
  }
  __syncthreads();
  return (int)uniform_u32((uint32_t)st->slot);
}

// Workgroups of Kernel (threads each, static LDS only) that the current
// device holds at once: the grid of a persistent launch (looked up once per
// device and kernel)
template <auto Kernel>
int resident_workgroups(int threads) {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  if (dev < 64 && cached[dev] > 0) return cached[dev];
  int cus = 0, per = 0;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, Kernel, threads, 0);
  const int n = cus * per > 0 ? cus * per : 1;
  if (dev < 64) cached[dev] = n;
  return n;
}

// zeroes the kQueueLanes work-queue counters of a persistent launch on its
// stream (a kernel, not a memset, so the launch pair can be captured in a
// graph)
static __global__ void zero_counter_kernel(int* counter) { counter[threadIdx.x] = 0; }

// The kernel's argument struct, re-read from the kernarg segment through a
// pointer the compiler cannot see through: a persistent kernel then reloads
// its arguments (scalar loads) per pair instead of holding them in SGPRs
// across the whole loop, where they spill.  A is the kernel's only argument.
template <class A>
__device__ __forceinline__ A kernel_args() {
#if __HIP_DEVICE_COMPILE__
  typedef __attribute__((address_space(4))) const A* cptr;
  cptr p = (cptr)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return *p;
#else
  return A{};  // (host pass; device code only)
#endif
}

// threadIdx.x as a value the compiler cannot see through: the lane-dependent
// offsets of a pair are then computed per pair, not hoisted out of a
// persistent kernel's loop to stay live (and spill) across it
__device__ __forceinline__ int opaque_thread_id() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// ------------------------------------------------------------ row tiles
// A bf16 tile [64][D] (rows of W = 2D bytes) is kept in LDS without padding,
// one quad of rows (4 rows, Q = 4W bytes) after the other, each quad being a
// permutation of the quad's Q contiguous bytes in memory, so one 1 KB
// DMA instruction copies whole contiguous rows.  Inside the quad of rows
// 4m .. 4m + 3, 16-byte chunk c of row 4m + k sits at byte
//     256 (c >> 2) + 64 k + 16 ((c & 3) ^ (m & 3)),
// so the 64-bank word address of a chunk is 4 k + ((c & 3) ^ (m & 3)) (mod 16
// chunk slots).  Two read patterns use the same tile without bank conflicts:
//  * RowOperand: an MFMA operand whose contraction runs along the tile's
//    columns (lane (l32, g) takes 8 elements of row R + l32 at column
//    16 s + 8 g) -- one ds_read_b128; the 16 lanes of one LDS cycle read 16
//    consecutive rows of one chunk, slots 4 (r & 3) + (((r >> 2) & 3) ^ c):
//    all distinct;
//  * TrOperand: an MFMA operand whose contraction runs along the tile's rows
//    (lane (l32, g) takes column 32 dt + l32 at the eight rows
//    16 tt + {4g .. 4g+3, 8+4g .. 8+4g+3}, the k-slot order of an operand
//    built from an accumulator, see b_from_acc) -- two ds_read_b64_tr_b16.
//    Within each 16-lane group, lane 16b + 4i + e of ds_read_b64_tr_b16
//    receives element e of the 8-byte chunks addressed by lanes 16b + 4k + i,
//    k = 0..3 (in slot k).  The 32 lanes of one LDS cycle read the four rows
//    of one quad at the four chunks 4 dt .. 4 dt + 3: slots 4 k + (x ^ m),
//    all distinct.
// Every per-step offset is a lane base plus an immediate, and the same tile
// serves S = Q K^T-type products and the transposed products (dK = dS^T Q,
// dQ = dS K, O = P V), so no transposed copies are needed.
template <int D>
struct RowTile {
  static constexpr int W = 2 * D, Q = 4 * W, BYTES = 64 * W, KB = BYTES / 1024;
  static_assert(BYTES % 1024 == 0 && (1024 % Q == 0 || Q % 1024 == 0), "quads tile whole KB");
  // byte offset of row R (a multiple of 4) in the tile
  static constexpr int rows(int R) { return (R >> 2) * Q; }
  // global byte offset fetched by lane `lane` of KB-instruction i of the tile.
  // Instructions i and i + 4m fetch at offsets 4096 m apart (the swizzle of a
  // quad depends on the quad index mod 4 only), so a wave that issues every
  // fourth instruction keeps one lane offset and advances the scalar base.
  static __device__ __forceinline__ uint32_t src_offset(int i, int lane) {
    const int pos = 1024 * i + 16 * lane;
    const int rq = pos / Q, rem = pos - rq * Q;
    const int k = (rem >> 6) & 3;
    const int c = 4 * (rem >> 8) + (((rem >> 4) & 3) ^ (rq & 3));
    return (uint32_t)((4 * rq + k) * W + 16 * c);
  }
};

struct RowOperand {
  uint32_t even, odd;  // byte offsets in the tile for even / odd k-steps s
  // rows R + l32 (R a multiple of 4, may be wave-uniform runtime)
  template <class RT>
  __device__ __forceinline__ void init(int R, int l32, int g) {
    const int r = R + l32, m = (r >> 2) & 3;
    const int base = (r >> 2) * RT::Q + 64 * (r & 3);
    even = (uint32_t)(base + 16 * (m ^ g));
    odd = (uint32_t)(base + 16 * (m ^ (2 + g)));
  }
  __device__ __forceinline__ bf16x8 load(const uint8_t* tile, int s) const {
    return *reinterpret_cast<const bf16x8*>(tile + ((s & 1) ? odd : even) + 256 * (s >> 1));
  }
};

typedef short prism_v4s __attribute__((ext_vector_type(4)));
typedef short prism_v8s __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) prism_v4s prism_lds_v4s;

struct TrOperand {
  uint32_t h0, h1;  // byte offsets of rows 16tt + 4g + k and 16tt + 8 + 4g + k (tt = 0)
  // R0: first tile row of k-step tt = 0 (a multiple of 4, may be wave-uniform)
  template <class RT>
  __device__ __forceinline__ void init(int R0, int lane) {
    const int b = lane >> 4, k = (lane >> 2) & 3, i = lane & 3;
    const int x = 2 * (b & 1) + (i >> 1);  // chunk of the lane within its 4-chunk group
    const int r0 = R0 + 4 * (b >> 1) + k, r1 = r0 + 8;
    h0 = (uint32_t)((r0 >> 2) * RT::Q + 64 * k + 16 * (((r0 >> 2) & 3) ^ x) + 8 * (i & 1));
    h1 = (uint32_t)((r1 >> 2) * RT::Q + 64 * k + 16 * (((r1 >> 2) & 3) ^ x) + 8 * (i & 1));
  }
  template <class RT>
  __device__ __forceinline__ bf16x8 load(const uint8_t* tile, int tt, int dt) const {
    const uint8_t* p0 = tile + h0 + 4 * RT::Q * tt + 256 * dt;
    const uint8_t* p1 = tile + h1 + 4 * RT::Q * tt + 256 * dt;
    const prism_v4s r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((prism_lds_v4s*)(p0));
    const prism_v4s r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((prism_lds_v4s*)(p1));
    const prism_v8s v = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(bf16x8, v);
  }
};
