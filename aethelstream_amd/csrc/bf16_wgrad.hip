// bf16_wgrad.hip - weight gradient dW = dY^T . X for gfx950 (MI355X).
//
//   dw[n, k] (+)= sum_m dy[m, n] * x[m, k]
// the d_wd / d_wg / d_wu / d_wo / d_wq / d_wk / d_wv loops of
// single_layer_backward (doublepass/src/backward.rs:87-93, 117-129, 160-168,
// 284-300), with the micro-batch accumulation of backward.rs:478-502 as the
// `accumulate` flag.  dy [M, N] and x [M, K] are bf16, row-major; dw [N, K]
// fp32.  The reduction runs over the token index m, the row index of both
// operands, so both MFMA operands are columns of row-major tiles.
//
// Workgroup = 4 waves in 2 x 2, tile = 256 dW rows (n) x 256 dW columns (k);
// each wave owns 128 x 128 in 256 accumulator registers (16 tiles of
// v_mfma_f32_32x32x16_bf16).  Per 32-token step the dy tile (32 x 256 bf16)
// and the x tile (32 x 256) move into LDS with direct-to-LDS loads, into a
// ring of kWgStages 32 KB stages that keeps the next kWgStages - 1 steps in
// flight while step t computes (3 stages measured faster than 2 of 64
// tokens, and than 4 or 5 of 32), and each wave reads its fragments with
// the transposing ds_read_b64_tr_b16: 8 consecutive tokens of one column
// per lane.
#include "abi_common.hpp"
#include "gemm_common.hpp"
#include "nf4_device.hpp"

namespace nf4s {

constexpr int kWgThreads = 256;
constexpr int kWgTile = 256;  // dW rows and columns per workgroup
constexpr int kWgStep = 32;   // tokens per step
constexpr int kWgStages = 3;  // LDS ring stages

constexpr int kMaxWgGroups = 4;  // products per launch that share x

// The products of one launch stack their dW row tiles: product i owns tile
// rows tile0[i] .. tile0[i+1]-1 of a tiles_n x tiles_k grid.
struct WgradArgs {
  const uint16_t *dy[kMaxWgGroups];  // [M, N_i], row stride N_i
  float *dw[kMaxWgGroups];           // [N_i, K], row stride K
  int64_t N[kMaxWgGroups];
  int32_t tile0[kMaxWgGroups + 1];
  int32_t ngroups;
  const uint16_t *x;  // [M, K], row stride K
  int64_t M, K;
  int32_t tiles_n, tiles_k;
  int32_t accumulate;
  int32_t blk_n, blk_k;  // XCD block of blk_n x blk_k tiles (0: map_tile order)
};

// a[i] for a wave-uniform i < kMaxWgGroups, as a chain of selects: indexing
// the kernel-argument arrays with a variable would copy them to scratch.
template <typename T>
__device__ __forceinline__ T wg_pick(const T (&a)[kMaxWgGroups], int i) {
  T v = a[0];
#pragma unroll
  for (int j = 1; j < kMaxWgGroups; ++j) v = (i == j) ? a[j] : v;
  return v;
}

// Tile order of a launch whose rounds are all full (T a multiple of the
// grid G, G / 8 slots per XCD): in round r, XCD x (workgroups b with
// b % 8 == x) takes block 8 r + x of blk_n x blk_k tiles, blk_n * blk_k =
// G / 8, slot i = (b % G) / 8 the tile (i / blk_k, i % blk_k) of the block.
// The XCD's workgroups then read blk_n dy column blocks and blk_k x column
// blocks per 64-token step (4 + 8 = 12 x 32 KB on a 256-CU part) instead of
// 1 + 32 in map_tile's order, where they share one dy block and read every
// x block of the row; the rest comes from the XCD's L2.
__device__ __forceinline__ void wg_map_tile(const WgradArgs &g, int b, int &tn, int &tk) {
  if (g.blk_n == 0) {
    map_tile(b, g.tiles_n, g.tiles_k, tn, tk);
    return;
  }
  const int G = gridDim.x;
  const int r = b / G, c = b - r * G;
  const int blk = 8 * r + (c & 7), i = c >> 3;
  const int nbk = g.tiles_k / g.blk_k;
  const int bn = blk / nbk, bk = blk - bn * nbk;
  tn = bn * g.blk_n + i / g.blk_k;
  tk = bk * g.blk_k + i % g.blk_k;
}

// LDS tile: 32 token rows x 256 columns (512 B = 32 units of 16 B per row).
// A wave reads one 128-column half (16 units).  Unit u of row r lives at
// physical unit (u & 16) | ((u & 15) ^ 5 (r % 4)): with it, each 32-lane
// half of a transposed fragment read covers 16 distinct 16-B units of one
// half-row's 64 banks (rows are 512 B = 128 banks apart, so every row starts
// at bank 0), and each 16-lane quarter of a DMA writes one row's 16
// contiguous units.
__device__ __forceinline__ int wg_unit(int row, int u) {
  return (u & 16) | ((u & 15) ^ (5 * (row & 3)));
}

// [stage][operand 0 = dy, 1 = x][row * 32 + unit]: kWgStages x 2 x 16 KB.
__shared__ u32x4 g_wg_lds[kWgStages][2][kWgStep * 32];

// Byte offset (from its tile's base) of lane `lane`'s first transposed read
// of fragment j: column 32j + lane % 32 of the wave's half h, token rows
// 8 (lane / 32) + 0..3 of sub-step 0.  ds_read_b64_tr_b16 transposes 4 x 4
// blocks of 16-bit values within each 16-lane group: lane i receives element
// i % 4 of the 8 bytes that lane 4e + i / 4 addresses, so lane 4e + c
// addresses row e, columns 4c..4c+3 of the group's 16-column strip.  A second
// read 4 rows lower completes the 8 tokens.
__device__ __forceinline__ uint32_t wg_read_off(int lane, int h, int j) {
  const int l16 = lane & 15, e = l16 >> 2;
  const int row = 8 * (lane >> 5) + e;
  const int u = 16 * h + 4 * j + 2 * ((lane >> 4) & 1) + ((l16 >> 1) & 1);
  return (uint32_t)(512 * row + 16 * wg_unit(row, u) + 8 * (l16 & 1));
}

// Fragment (8 tokens of one column, sub-step s) from the tile at `base`.
__device__ __forceinline__ u32x4 wg_frag(const char *base, uint32_t off, int s) {
  typedef __attribute__((address_space(3))) char lds_char_t;
  typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
  lds_char_t *p = (lds_char_t *)const_cast<char *>(base) + off + 8192 * s;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)p);
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(p + 2048));
  const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
  return (u32x4){l2.x, l2.y, h2.x, h2.y};
}

// Fragment read q (0..7) of a sub-step in the order the sub-step's first
// MFMAs use them: dy0, x0, x1, x2, x3, dy1, dy2, dy3.
__device__ __forceinline__ void wg_read(const char *tdy, const char *tx, const uint32_t (&rdy)[4],
                                        const uint32_t (&rx)[4], u32x4 (&fd)[4], u32x4 (&fx)[4],
                                        int s, int q) {
  if (q == 0 || q >= 5) {
    const int j = (q == 0) ? 0 : q - 4;
    fd[j] = wg_frag(tdy, rdy[j], s);
  } else {
    fx[q - 1] = wg_frag(tx, rx[q - 1], s);
  }
}

// One 32-token step t from stage `cur`: 2 sub-steps of 16 MFMAs.  The
// fragments of sub-step 1 are read (one per MFMA slot) during sub-step 0.
// The 8 DMAs of this wave for step t + kWgStages - 1 (4 dy row pairs, 4 x
// row pairs, two 256-column rows per instruction) go into stage `nxt` after
// MFMAs 9, 11, .., 23 (the same DMAs in sub-step 0's first half measured
// 1-2 % slower on 70B shapes); that stage held step t-1, whose reads all
// ended before the barrier that closed step t-1.  The caller's barrier
// after MFMA 7 of sub-step 1 waits for step t+1's DMAs (leaving the later
// steps' in flight) and every LDS read; the last 8 MFMAs (operands in
// registers) open the next call, each followed by one of the next step's
// sub-step 0 reads.
// `more` (that step exists) is a branch around the DMAs, which keeps each
// DMA after its slot's MFMA and reads.  The LDS stages come in as distinct
// __restrict__ pointers: the compiler then knows that DMAs into `nxt` never
// alias the reads of `cur` and waits (vmcnt) only at the barriers.
__device__ __forceinline__ void wgrad_step(floatx16 (&acc)[4][4], u32x4 (&fd)[2][4],
                                           u32x4 (&fx)[2][4], const char *__restrict__ cur_dy,
                                           const char *__restrict__ cur_x,
                                           char *__restrict__ nxt_dy, char *__restrict__ nxt_x,
                                           const uint32_t (&rdy)[4], const uint32_t (&rx)[4],
                                           __amdgpu_buffer_rsrc_t rs_dy, __amdgpu_buffer_rsrc_t rs_x,
                                           uint32_t (&vdy)[4], uint32_t (&vx)[4],
                                           uint32_t step_dy, uint32_t step_x, bool more, int wave) {
  // Previous step's last 8 MFMAs, then this step's sub-step 0 reads.
  static_for<0, 8>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int mt = 2 + (i >> 2), nt = i & 3;
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, fx[1][nt]), __builtin_bit_cast(bf16x8, fd[1][mt]),
        acc[mt][nt], 0, 0, 0);
    wg_read(cur_dy, cur_x, rdy, rx, fd[0], fx[0], 0, i);
    __builtin_amdgcn_sched_barrier(0);
  });
  static_for<0, 24>([&](auto N) {
    constexpr int n = decltype(N)::value;
    constexpr int s = n / 16, i = n % 16;
    constexpr int mt = i >> 2, nt = i & 3;
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, fx[s][nt]), __builtin_bit_cast(bf16x8, fd[s][mt]),
        acc[mt][nt], 0, 0, 0);
    if constexpr (s == 0 && i < 8) wg_read(cur_dy, cur_x, rdy, rx, fd[1], fx[1], 1, i);
    if constexpr (n >= 8 && (n & 1) == 1) {
      // DMA d = (n - 8) / 2 after MFMAs 9, 11, .., 23: operand d / 4,
      // instruction d % 4 (rows 8 wave + 2 (d % 4) and the next).
      constexpr int d = (n - 8) / 2;
      if (more) {
        if constexpr (d < 4) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs_dy, (lds_void_t *)(nxt_dy + 1024 * (4 * wave + d)), 16,
              (int)vdy[d], 0, 0, 0);
          vdy[d] += step_dy;
        } else {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs_x, (lds_void_t *)(nxt_x + 1024 * (4 * wave + d - 4)), 16, (int)vx[d - 4], 0, 0,
              0);
          vx[d - 4] += step_x;
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  });
}

// The barrier that closes step t: this wave's DMAs of step t+1 have landed
// and every LDS read of step t has ended.  Its DMAs of the later steps in
// the ring (t+2 .. t+kWgStages-1, 8 each, issued after t+1's, those that
// exist) may still be in flight: vmcnt retires in issue order.
__device__ __forceinline__ void wgrad_close_step(int64_t t, int64_t nsteps) {
  int64_t later = nsteps - t - 2;  // steps after t+1 that exist, clamped below
  later = (later < 0) ? 0 : (later > kWgStages - 2) ? kWgStages - 2 : later;
  static_for<0, kWgStages - 1>([&](auto I) {
    constexpr int a = decltype(I)::value;  // exactly one a == later
    if (later == a) step_barrier<8 * a>();
  });
}

// One output tile: its 256 x 256 dW block over all M tokens.
__global__ void __launch_bounds__(kWgThreads, 1) wgrad_kernel(const WgradArgs g) {
  const int T = g.tiles_n * g.tiles_k;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int hn = wave >> 1, hk = wave & 1;  // the wave's halves of n and k
  uint32_t rdy[4], rx[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    rdy[j] = wg_read_off(lane, hn, j);
    rx[j] = wg_read_off(lane, hk, j);
  }
  char *ldy[kWgStages], *lx[kWgStages];
#pragma unroll
  for (int i = 0; i < kWgStages; ++i) {
    ldy[i] = reinterpret_cast<char *>(&g_wg_lds[i][0][0]);
    lx[i] = reinterpret_cast<char *>(&g_wg_lds[i][1][0]);
  }
  const int64_t nsteps = (g.M + kWgStep - 1) / kWgStep;
  const uint32_t step_x = (uint32_t)(kWgStep * g.K * 2);
#pragma unroll 1
  for (int b = blockIdx.x; b < T; b += gridDim.x) {
    int tn, tk;
    wg_map_tile(g, b, tn, tk);
    // The product that owns tile row tn.
    int gi = 0;
#pragma unroll
    for (int j = 1; j < kMaxWgGroups; ++j) gi += (j < g.ngroups && tn >= g.tile0[j]) ? 1 : 0;
    const uint16_t *dy = wg_pick(g.dy, gi);
    float *dw = wg_pick(g.dw, gi);
    const int64_t N = wg_pick(g.N, gi);
    int32_t t0 = g.tile0[0];
#pragma unroll
    for (int j = 1; j < kMaxWgGroups; ++j) t0 = (gi == j) ? g.tile0[j] : t0;
    const int64_t n0 = (int64_t)(tn - t0) * kWgTile, k0 = (int64_t)tk * kWgTile;
    const uint32_t step_dy = (uint32_t)(kWgStep * N * 2);
    // Buffer resources based at the tiles' first columns; num_records ends
    // at the matrix end, so token rows >= M (and the last row's columns past
    // the end) read as zero.  Columns past N or K of other rows read the next
    // row's values and only reach outputs that are never stored.
    const __amdgpu_buffer_rsrc_t rs_dy = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(dy + n0), 0, (int)(g.M * N * 2 - n0 * 2), kBufferFlags);
    const __amdgpu_buffer_rsrc_t rs_x = __builtin_amdgcn_make_buffer_rsrc(
        (void *)(g.x + k0), 0, (int)(g.M * g.K * 2 - k0 * 2), kBufferFlags);
    // Lane offsets of this wave's 4 DMAs per operand for step 0: instruction
    // d writes rows 8 wave + 2d + (lane / 32), physical unit lane % 32.
    uint32_t vdy[4], vx[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const int r = 8 * wave + 2 * d + (lane >> 5);
      const int u = wg_unit(r, lane & 31);  // the logical unit stored at physical lane % 32
      vdy[d] = (uint32_t)(r * N * 2 + 16 * u);
      vx[d] = (uint32_t)(r * g.K * 2 + 16 * u);
    }
    // Prologue: steps 0 .. kWgStages-2 (those that exist) into their
    // stages, then wait for step 0.
#pragma unroll
    for (int p = 0; p < kWgStages - 1; ++p) {
      if (p < nsteps) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs_dy, (lds_void_t *)(ldy[p] + 1024 * (4 * wave + d)), 16, (int)vdy[d], 0, 0, 0);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(
              rs_x, (lds_void_t *)(lx[p] + 1024 * (4 * wave + d)), 16, (int)vx[d], 0, 0, 0);
          vdy[d] += step_dy;
          vx[d] += step_x;
        }
      }
    }
    wgrad_close_step(-1, nsteps);

    floatx16 acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[mt][nt][v] = 0.0f;
    u32x4 fd[2][4], fx[2][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      fd[1][i] = (u32x4){0u, 0u, 0u, 0u};
      fx[1][i] = (u32x4){0u, 0u, 0u, 0u};
    }
    // Step t computes from stage t % kWgStages and loads step
    // t + kWgStages - 1 into the stage before it.
    int64_t t = 0;
#pragma unroll 1
    for (; t + kWgStages <= nsteps; t += kWgStages) {
      static_for<0, kWgStages>([&](auto I) {
        constexpr int i = decltype(I)::value;
        constexpr int c = i, nx = (i + kWgStages - 1) % kWgStages;
        wgrad_step(acc, fd, fx, ldy[c], lx[c], ldy[nx], lx[nx], rdy, rx, rs_dy, rs_x, vdy, vx,
                   step_dy, step_x, t + i + kWgStages - 1 < nsteps, wave);
        wgrad_close_step(t + i, nsteps);
      });
    }
    static_for<0, kWgStages - 1>([&](auto I) {
      constexpr int i = decltype(I)::value;
      constexpr int c = i, nx = (i + kWgStages - 1) % kWgStages;
      if (t + i < nsteps) {
        wgrad_step(acc, fd, fx, ldy[c], lx[c], ldy[nx], lx[nx], rdy, rx, rs_dy, rs_x, vdy, vx,
                   step_dy, step_x, false, wave);
        wgrad_close_step(t + i, nsteps);
      }
    });
    // The last step's final 8 MFMAs.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int mt = 2 + (i >> 2), nt = i & 3;
      acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          __builtin_bit_cast(bf16x8, fx[1][nt]), __builtin_bit_cast(bf16x8, fd[1][mt]),
          acc[mt][nt], 0, 0, 0);
    }

    // Epilogue.  Lane l holds dW row n = n0 + 128 hn + 32 mt + l % 32 and
    // columns k = k0 + 128 hk + 32 nt + 8 j + 4 (l / 32) + i in registers
    // 4 j + i of tile [mt][nt]: four adjacent fp32 per 16-B store.
    const int jl = lane & 31, grp = lane >> 5;
    const bool vec_ok = ((reinterpret_cast<uintptr_t>(dw) & 15) == 0) && ((g.K & 3) == 0);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      const int64_t n = n0 + 128 * hn + 32 * mt + jl;
      if (n < N) {
        float *row = dw + n * g.K;
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int64_t k = k0 + 128 * hk + 32 * nt + 8 * j + 4 * grp;
            floatx4 v = {acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1], acc[mt][nt][4 * j + 2],
                         acc[mt][nt][4 * j + 3]};
            if (vec_ok && k + 4 <= g.K) {
              floatx4 *p = reinterpret_cast<floatx4 *>(row + k);
              if (g.accumulate) v += *p;
              *p = v;
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i)
                if (k + i < g.K) row[k + i] = g.accumulate ? row[k + i] + v[i] : v[i];
            }
          }
      }
    }
    // The next tile's prologue DMAs overwrite stage 0, which the last
    // step's reads may have used: every wave's reads end before this.
    step_barrier<0>();
  }
}

__global__ void fill_zero_f32(float *__restrict__ p, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

static int32_t wgrad_grouped(const uint16_t *const *dys, const int64_t *ns, float *const *dws,
                             int32_t count, const uint16_t *x, int64_t m, int64_t k,
                             int32_t accumulate, hipStream_t s) {
  if (count < 1 || count > kMaxWgGroups)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "weight-gradient product count %d outside [1, %d]",
                count, kMaxWgGroups);
  if (dys == nullptr || ns == nullptr || dws == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "dys, ns or dws is NULL");
  if (m < 0 || k <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad weight-gradient shape m=%lld k=%lld",
                (long long)m, (long long)k);
  constexpr int64_t kMaxDim = (int64_t)1 << 39;  // tile counts below are 32-bit
  if (k > kMaxDim)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "weight-gradient k=%lld beyond 2^39", (long long)k);
  if (k % 8 != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "weight gradient needs k %% 8 == 0, got k=%lld",
                (long long)k);
  if (m > 0 && x == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "x is NULL");
  if (m > 0 && !aligned(x, 16)) return fail(NF4S_ERR_MISALIGNED, "x must be 16-byte aligned");
  // Lane offsets are 32-bit and must stay below 2^31 for every row a step
  // addresses, including the rows past m of the last 32-token step (which
  // read as zero only while their offsets do not wrap onto real rows).
  // The comparisons divide instead of multiplying, so no caller size can
  // overflow them.
  const int64_t lim = ((int64_t)1 << 31) - 1;
  const int64_t rows = m / kWgStep * kWgStep + (m % kWgStep ? kWgStep : 0);
  if (rows > 0 && k > lim / 2 / rows)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                "x larger than 2 GiB with m rounded up to 32 (m=%lld k=%lld)", (long long)m,
                (long long)k);
  WgradArgs g{};
  g.ngroups = count;
  g.x = x;
  g.M = m;
  g.K = k;
  g.tiles_k = (int32_t)((k + kWgTile - 1) / kWgTile);
  g.accumulate = accumulate ? 1 : 0;
  int64_t tiles_n = 0;
  for (int i = 0; i < count; ++i) {
    const int64_t n = ns[i];
    if (dws[i] == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "dw %d is NULL", i);
    if (m > 0 && dys[i] == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "dy %d is NULL", i);
    if (n <= 0)
      return fail(NF4S_ERR_INVALID_ARGUMENT, "bad weight-gradient shape m=%lld n=%lld k=%lld",
                  (long long)m, (long long)n, (long long)k);
    if (n > kMaxDim)
      return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "weight-gradient n=%lld beyond 2^39", (long long)n);
    if (n % 8 != 0)
      return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "weight gradient needs n %% 8 == 0 and k %% 8 == 0, "
                  "got n=%lld k=%lld", (long long)n, (long long)k);
    if (m > 0 && !aligned(dys[i], 16))
      return fail(NF4S_ERR_MISALIGNED, "dy and x must be 16-byte aligned");
    if (!aligned(dws[i], 4)) return fail(NF4S_ERR_MISALIGNED, "dw must be 4-byte aligned");
    int64_t nk;
    if (__builtin_mul_overflow(n, k, &nk))
      return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "dW of %lld x %lld elements overflows 64 bits",
                  (long long)n, (long long)k);
    if (rows > 0 && n > lim / 2 / rows)
      return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                  "dy or x larger than 2 GiB with m rounded up to 32 (m=%lld n=%lld k=%lld)",
                  (long long)m, (long long)n, (long long)k);
    g.dy[i] = dys[i];
    g.dw[i] = dws[i];
    g.N[i] = n;
    g.tile0[i] = (int32_t)tiles_n;
    tiles_n += (n + kWgTile - 1) / kWgTile;
    if (tiles_n > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
  }
  for (int i = count; i <= kMaxWgGroups; ++i) g.tile0[i] = (int32_t)tiles_n;
  g.tiles_n = (int32_t)tiles_n;
  const int64_t T = tiles_n * g.tiles_k;
  if (T > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
  if (m == 0) {
    // An empty sum: dw += 0, or dw = 0 (a fill kernel rather than
    // hipMemsetAsync, so that a caller may capture the call in a HIP graph).
    // The main kernel's buffer bounds assume m > 0.
    if (accumulate) return NF4S_OK;
    for (int i = 0; i < count; ++i) {
      const int64_t cnt = ns[i] * k;
      const int64_t blocks = (cnt + 255) / 256;
      hipLaunchKernelGGL(fill_zero_f32, dim3((uint32_t)(blocks < 65536 ? blocks : 65536)),
                         dim3(256), 0, s, dws[i], cnt);
      const int32_t rc = check_launch("fill_zero_f32");
      if (rc != NF4S_OK) return rc;
    }
    return NF4S_OK;
  }
  // XCD blocks (wg_map_tile) when every round is full: the squarest
  // blk_n x blk_k = G / 8 that divides the tile grid (the products' tile
  // rows stacked).
  const int64_t G = persistent_grid(T);
  if (G % 8 == 0 && T % G == 0) {
    const int S = (int)(G / 8);
    int best = 0;
    for (int bn = 1; bn <= S; ++bn) {
      if (S % bn != 0 || g.tiles_n % bn != 0 || g.tiles_k % (S / bn) != 0) continue;
      const int bk = S / bn;
      const int cost = bn + bk;  // column blocks read per XCD and step
      if (best == 0 || cost < best) {
        best = cost;
        g.blk_n = bn;
        g.blk_k = bk;
      }
    }
  }
  hipLaunchKernelGGL(wgrad_kernel, dim3((uint32_t)G), dim3(kWgThreads), 0, s, g);
  return check_launch("wgrad_kernel");
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

int32_t nf4s_gemm_wgrad(const void *dy, const void *x, int64_t m, int64_t n, int64_t k,
                        float *dw, int32_t accumulate, void *stream) {
  clear_error();
  const uint16_t *dys[1] = {static_cast<const uint16_t *>(dy)};
  float *dws[1] = {dw};
  return wgrad_grouped(dys, &n, dws, 1, static_cast<const uint16_t *>(x), m, k, accumulate,
                       as_stream(stream));
}

int32_t nf4s_gemm_wgrad_grouped(const void *const *dys, const int64_t *ns, float *const *dws,
                                int32_t count, const void *x, int64_t m, int64_t k,
                                int32_t accumulate, void *stream) {
  clear_error();
  return wgrad_grouped(reinterpret_cast<const uint16_t *const *>(dys), ns, dws, count,
                       static_cast<const uint16_t *>(x), m, k, accumulate, as_stream(stream));
}

}  // extern "C"
