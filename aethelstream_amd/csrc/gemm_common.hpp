// gemm_common.hpp - pieces shared by the MFMA GEMM kernels for gfx950: vector
// types, compile-time loops, s_waitcnt encodings, the step barrier, the
// XCD-aware tile order and the persistent grid size.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace nf4s {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

typedef __attribute__((address_space(3))) void lds_void_t;

// Compile-time loop: f(IC<B>{}), ..., f(IC<E-1>{}).  Slot plans, fragment
// indices and LDS immediate offsets are then constant expressions.
template <int N>
struct IC {
  static constexpr int value = N;
};
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(IC<B>{});
    static_for<B + 1, E>(f);
  }
}

// Word 3 of a raw (stride 0) gfx9 buffer resource: 32-bit data format.
constexpr int kBufferFlags = 0x00020000;

// s_waitcnt immediates (gfx9 encoding: vmcnt[3:0] | expcnt[6:4] |
// lgkmcnt[11:8] | vmcnt[5:4] << 14).
constexpr int kWaitLgkm0 = 0xC07F;       // lgkmcnt(0), vmcnt and expcnt not waited
// vmcnt(n) lgkmcnt(0), expcnt not waited.
constexpr int wait_vm_lgkm0(int n) { return (n & 15) | 0x70 | ((n >> 4) << 14); }

// Workgroup barrier without the memory-model fences of __syncthreads(): the
// release fence would wait for every outstanding load (vmcnt(0)), including
// the DMAs that are meant to stay in flight across it.  The waits the
// barrier needs are issued explicitly before it (all but the kInFlight most
// recent vector-memory operations, and every LDS operation); the empty asm
// keeps the compiler from moving memory operations across it.
template <int kInFlight>
__device__ __forceinline__ void step_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(wait_vm_lgkm0(kInFlight));
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Maps tile index b to (tile_m, tile_o).  Workgroups are dispatched
// round-robin over the 8 XCDs and the persistent grid is a multiple of 8, so
// tile b runs on XCD b % 8; consecutive logical tiles (same tile_m,
// neighbouring tile_o) are given to the same XCD so that its resident
// workgroups share the tile_m operand rows in that XCD's L2.
//
// Exception: with 64 output tiles per row block (a 256-CU round covers 4
// row blocks) XCD pair (x, x + 4) shares one row block per round, each XCD
// taking 32 of its output tiles: tm = 4r + x % 4, to = 32 (x / 4) + i for
// round r and slot i.  Both XCDs then read those activation rows at the
// same time, and the Infinity Cache serves the second; in the XCD-major
// order one XCD reads them twice, a round apart.  A permutation of
// [0, tiles_m * 64) for any grid; measured +1.8 % on the 70B down
// projection (K = 28672, a 470 MB activation), +0.3 % on 70B q.
__device__ __forceinline__ void map_tile(int b, int tiles_m, int tiles_o, int &tm, int &to) {
  if (tiles_o == 64 && (tiles_m & 3) == 0) {
    const int r = b >> 8, x = b & 7, i = (b & 255) >> 3;
    tm = 4 * r + (x & 3);
    to = 32 * (x >> 2) + i;
    return;
  }
  const int T = tiles_m * tiles_o;
  const int x = b & 7, qq = b >> 3;
  const int base = T >> 3, rem = T & 7;
  const int L = x * base + (x < rem ? x : rem) + qq;
  tm = L / tiles_o;
  to = L - tm * tiles_o;
}

// Persistent grid: one workgroup per compute unit (a workgroup takes all or
// most of a CU's LDS), each looping over tiles b, b + grid, ...  A tile's
// output stores then drain while the same workgroup's next tile starts
// loading.  The CU count is read once per device; a multiple of 8 keeps tile
// b on XCD b % 8 (map_tile).
// The current device's compute-unit count rounded up to a multiple of 8.
inline int cu_slots() {
  static std::atomic<int> cus[64];  // zero-initialized (static storage)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int c = cus[dev].load(std::memory_order_relaxed);
  if (c == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0)
      n = 256;
    c = (n + 7) & ~7;
    cus[dev].store(c, std::memory_order_relaxed);  // every caller stores the same value
  }
  return c;
}

inline uint32_t persistent_grid(int64_t tiles) {
  const int c = cu_slots();
  return (uint32_t)(tiles < c ? tiles : c);
}

}  // namespace nf4s
