// nf4_gemm.hip - NF4-dequant-fused bf16 GEMM for gfx950 (MI355X).
//
//   forward  y[m,n]  = x[m,k]  . W^T   (matmul_tb, doublepass/src/math.rs:9-21)
//   dgrad    dx[m,k] = dy[m,n] . W     (doublepass/src/backward.rs:79-85, ...)
// with W [n,k] NF4 (blocks of 64 along k, fp32 or double-quantized absmax),
// bf16 activations, fp32 accumulation in v_mfma_f32_32x32x16_bf16, bf16 out.
//
// Workgroup = 4 waves, tile = 512 rows of the activation x 128 output columns.
// Each wave owns 128 rows and keeps a 128x128 fp32 accumulator (16 MFMA
// tiles of 32x32, 256 registers).  Per 64-deep reduction step:
//   * each wave moves its next activation tile (128 rows x 64 bf16) from
//     global memory into its own LDS buffer with direct-to-LDS loads, each
//     instruction one coalesced 1 KB run of 8 whole rows; the MFMA fragments
//     are then read from LDS;
//   * the workgroup dequantizes the step's 128x64 weight tile ONCE into LDS
//     as bf16 (16-entry per-block product table in registers, v_perm_b32
//     lookups), so the dequant cost is amortised over 512 activation rows;
//   * all 4 waves read the weight fragments from LDS and issue 64 MFMAs.
// The weight tile of step t+1 is dequantized while step t's MFMAs run (two
// LDS buffers, one workgroup barrier per step).
//
// MFMA operand layout used (32x32x16): lane l supplies row / column l % 32
// and 8 reduction slots from lane group g = l / 32.  The kernel assigns
// reduction index 32g + 8s + e to slot e of sub-step s for BOTH operands, so
// a lane's 4 sub-steps read 64 contiguous bytes of its activation row.  The
// accumulator layout is lane l: column l % 32, row 8(v/4) + 4g + v%4; the
// weight fragment is the first operand, so the accumulator's columns are
// activation rows and its rows are output columns.
#include "abi_common.hpp"
#include "nf4_device.hpp"

namespace nf4s {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int kGemmThreads = 256;
constexpr int kTileM = 512;   // activation rows per workgroup (128 per wave)
constexpr int kTileO = 128;   // output columns per workgroup
constexpr int kStep = 64;     // reduction depth per step (= NF4 block size)

struct GemmArgs {
  const uint16_t *a;  // activation [M, R] row-major (x or dy)
  int64_t lda;
  uint16_t *out;      // [M, O] row-major (y or dx)
  int64_t ldo;
  int64_t M, O, R;    // rows, output columns, reduction length
  const uint8_t *packed;
  AbsmaxRef am;
  int64_t wk;         // columns of W (its k); W row stride = wk/2 bytes
  int64_t wn;         // rows of W (its n)
  int32_t tiles_m, tiles_o;
};

// LDS tile: 128 rows x 64 bf16 (128 B = 8 units of 16 B).  Unit u of row r
// lives at r*8 + (u ^ (r & 7)) so that the 32 rows a wave reads for one
// fragment spread over all banks.
__device__ __forceinline__ int lds_unit(int row, int u) { return row * 8 + (u ^ (row & 7)); }

// Weight tile: the same swizzle XOR 2 * ((row / 32) % 4).  The extra term is
// constant over the 32 rows of one fragment read, so reads stay spread over
// the banks, and it spreads the dgrad producer's 16-bit stores (whose lanes
// cover output columns 32 apart) over all banks too.
__device__ __forceinline__ int lds_unit_b(int row, int u) {
  return row * 8 + (u ^ (row & 7) ^ ((row >> 4) & 6));
}

// Lookup of packed word w with product table t, finished by the producer's
// merge.
template <class Producer>
__device__ __forceinline__ void dequant_word(const Lut16 &t, uint32_t w, uint32_t out[4]) {
  WordLookup x;
  word_select(w, x);
  word_even(t, x);
  word_odd(t, x);
  Producer::merge(x, out);
}

// Absmax of block `blk`: fp32, or the double-quant code times its group
// scale.  It is loaded as raw words and decoded a step later, so that the
// loads' latency never stalls the wave.  A template flag rather than a
// runtime test keeps the GEMM step one basic block (one scheduling region).
struct AbsRaw {
  float s;     // fp32 absmax, or the group scale
  uint32_t q;  // double-quant code (0 without double-quant)
};

template <bool kDQ>
__device__ __forceinline__ AbsRaw absmax_load(const AbsmaxRef &a, int64_t blk) {
  AbsRaw r;
  if (kDQ) {
    r.q = a.q[blk];
    r.s = a.scale[blk >> a.group_shift];
  } else {
    r.q = 0;
    r.s = a.absmax[blk];
  }
  return r;
}

template <bool kDQ>
__device__ __forceinline__ float absmax_value(const AbsRaw &r) {
  return kDQ ? (float)r.q * r.s : r.s;
}

// Forward producer: thread -> (row n_local = tid/2, half h = tid%2), 32
// consecutive k of one block; writes 4 swizzled 16-B units of its row.
template <bool kDQ>
struct FwdProducer {
  const uint8_t *ptr;   // packed bytes of (row, half) at step 0
  int64_t am_idx;       // absmax block index at step 0
  int row, h;
  __device__ void init(const GemmArgs &g, int64_t o0) {
    row = threadIdx.x >> 1;
    h = threadIdx.x & 1;
    int64_t n = o0 + row;
    if (n >= g.wn) n = g.wn - 1;  // ragged N: clamp (outputs are not stored)
    ptr = g.packed + n * (g.wk >> 1) + 16 * h;
    am_idx = n * (g.wk >> 6);
  }
  __device__ __forceinline__ void load(const GemmArgs &g, int64_t step, u32x4 &w, AbsRaw &a) const {
    w = *reinterpret_cast<const u32x4 *>(ptr + step * 32);
    a = absmax_load<kDQ>(g.am, am_idx + step);
  }
  // The absmax the product table is built from.
  __device__ __forceinline__ float table_absmax(const AbsRaw &a) const {
    return absmax_value<kDQ>(a);
  }
  // The 8 elements of a word in natural order: out[j] = elements 2j, 2j+1.
  static __device__ __forceinline__ void merge(const WordLookup &x, uint32_t out[4]) {
    word_merge(x, out);
  }
  // Writes the 8 dequantized elements of packed word k in `part` of
  // kStoreParts.
  static constexpr int kStoreParts = 1;
  __device__ __forceinline__ void store(u32x4 *lds, const uint32_t out[4], int k, int part) const {
    (void)part;
    u32x4 v;
    v.x = out[0]; v.y = out[1]; v.z = out[2]; v.w = out[3];
    lds[lds_unit_b(row, 4 * h + k)] = v;
  }
  // Whole-tile store (prologue).
  __device__ __forceinline__ void store(u32x4 *lds, const u32x4 &w, const AbsRaw &a) const {
    const Lut16 lut = make_lut<false>(table_absmax(a));
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t o[4];
      dequant_word<FwdProducer>(lut, words[k], o);
      store(lds, o, k, 0);
    }
  }
};

// Dgrad producer: the step covers W rows n0..n0+63 (the reduction) and W
// columns o0..o0+127 (the output).  Thread -> (W row r = tid/4, quarter
// q = tid%4): 32 consecutive columns of one block.  The LDS tile is stored
// transposed (LDS row = output column, 64 reduction values per row), so
// each element is written as one 16-bit value.
template <bool kDQ>
struct DgradProducer {
  const uint8_t *ptr;
  int64_t am_idx;
  int r, q;
  uint32_t valid_mask;  // all ones when the thread's columns exist
  __device__ void init(const GemmArgs &g, int64_t o0) {
    r = threadIdx.x >> 2;
    q = threadIdx.x & 3;
    const int64_t col = o0 + 32 * q;
    const bool valid = col < g.wk;
    valid_mask = valid ? 0xffffffffu : 0u;
    const int64_t c = valid ? col : 0;
    ptr = g.packed + (int64_t)r * (g.wk >> 1) + (c >> 1);
    am_idx = (int64_t)r * (g.wk >> 6) + (c >> 6);
  }
  __device__ __forceinline__ void load(const GemmArgs &g, int64_t step, u32x4 &w, AbsRaw &a) const {
    // Step s covers W rows 64s .. 64s+63.
    w = *reinterpret_cast<const u32x4 *>(ptr + step * 64 * (g.wk >> 1));
    a = absmax_load<kDQ>(g.am, am_idx + step * 64 * (g.wk >> 6));
  }
  // Columns beyond k read column 0's bytes and are zeroed via the absmax.
  __device__ __forceinline__ float table_absmax(const AbsRaw &a) const {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, absmax_value<kDQ>(a)) & valid_mask);
  }
  // Elements are stored one by one, so the pairs of the first merge half
  // suffice: element j is half (j >> 1) & 1 of out[(j & 1) + 2 * (j >> 2)].
  static __device__ __forceinline__ void merge(const WordLookup &x, uint32_t out[4]) {
    word_pairs(x, out);
  }
  // Writes the 8 elements of packed word k as 16-bit values down 8 LDS rows
  // (output columns); part p of 4 writes elements 2p and 2p+1.
  static constexpr int kStoreParts = 4;
  __device__ __forceinline__ void store(u32x4 *lds, const uint32_t out[4], int k, int part) const {
    uint16_t *l16 = reinterpret_cast<uint16_t *>(lds);
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const int j = 2 * part + jj;
      const int col = 32 * q + 8 * k + j;  // LDS row (output column)
      const uint32_t pr = out[(j & 1) + 2 * (j >> 2)];
      const uint16_t v = (uint16_t)(((j >> 1) & 1) ? (pr >> 16) : (pr & 0xffffu));
      l16[lds_unit_b(col, r >> 3) * 8 + (r & 7)] = v;
    }
  }
  __device__ __forceinline__ void store(u32x4 *lds, const u32x4 &w, const AbsRaw &a) const {
    const Lut16 lut = make_lut<false>(table_absmax(a));
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t o[4];
      dequant_word<DgradProducer>(lut, words[k], o);
#pragma unroll
      for (int p = 0; p < 4; ++p) store(lds, o, k, p);
    }
  }
};

// Maps the workgroup index to (tile_m, tile_o).  Workgroups are dispatched
// round-robin over the 8 XCDs; consecutive logical tiles (same activation
// rows, neighbouring output columns) are given to the same XCD so that its
// resident workgroups share the activation rows in that XCD's L2.
__device__ __forceinline__ void map_tile(int tiles_m, int tiles_o, int &tm, int &to) {
  const int T = tiles_m * tiles_o;
  const int b = blockIdx.x;
  const int x = b & 7, qq = b >> 3;
  const int base = T >> 3, rem = T & 7;
  const int L = x * base + (x < rem ? x : rem) + qq;
  tm = L / tiles_o;
  to = L - tm * tiles_o;
}

// LDS: two activation buffers per wave (128 rows x 128 B = 16 KB each, a
// wave's pair adjacent) and two weight tiles (16 KB each): 160 KB, the gfx950
// maximum.  With the buffers of a pair 16 KB apart, the main loop (unrolled
// by two steps) addresses both through the LDS instructions' immediate
// offsets from loop-invariant lane addresses.
__shared__ u32x4 g_lds_a[4][2][1024];
__shared__ u32x4 g_lds_b[2][1024];

typedef __attribute__((address_space(3))) void lds_void_t;

// Word 3 of a raw (stride 0) gfx9 buffer resource: 32-bit data format.
constexpr int kBufferFlags = 0x00020000;

// One 64-deep reduction step: 4 sub-steps of 16 MFMAs over the activation
// tile in Acur (this wave's rows) and the weight tile in Bcur.  Alongside it
//   * starts the direct-to-LDS loads of the next step's activation tile into
//     Anext (16 instructions of 1 KB, 8 full 128-B rows each),
//   * loads the packed weight bytes of step t+2 (wn_, an_),
//   * dequantizes step t+1's weights (wc, ac) into Bnext,
//   * prefetches the next sub-step's A and B fragments.
// A wave issues in order, so other work only overlaps the matrix pipe when
// it sits between MFMAs in the instruction stream: every MFMA is followed by
// one small piece of that work (a few VALU ops, two LDS reads, a DMA), and
// sched_barrier fences keep that order.
//
// The step ends at the workgroup barrier after MFMA 11 of sub-step 3; its
// last 4 MFMAs (a[1][3] x b[1][0..3], operands already in registers) open
// the NEXT call, after the barrier, each followed by one pair of fragment
// reads of the new step's sub-step 0, so those reads' latency hides behind
// matrix work.  The first call runs them on zero operands.
//
// Slot plan, after MFMA i of sub-step s (R = fragment-read pair for s+1,
// D = activation DMA, L = product-table quarter, W = lookup stage of a
// packed word, P = part of a word's 16-bit transposed store):
//   s=0: i0-3 R + D0-3   i4-7 L0-3     i8-11 W(0)    i12-15 D4-7
//   s=1: i0-3 R + D8-11  i4-7 W(1)     i8-11 P(0)    i12-15 D12-15
//   s=2: i0-3 R          i4-7 W(2)     i8-11 P(1)
//   s=3: i0-3 P(2)       i4-7 W(3)     i8-11 P(3)    -> barrier
// The forward producer (no P jobs) issues its DMAs in slots 8-15 of
// sub-steps 0 and 1 instead, away from the fragment reads (measured faster
// for the forward, slower for dgrad).  The DMAs are all issued by the middle of the
// step, so they have landed by the barrier.
template <class Producer>
__device__ __forceinline__ void gemm_step(const GemmArgs &g, const Producer &prod,
                                          floatx16 (&acc)[4][4], u32x4 (&a)[2][4],
                                          u32x4 (&b)[2][4], const u32x4 *__restrict__ Acur,
                                          u32x4 *__restrict__ Anext_wave,
                                          const u32x4 *__restrict__ Bcur,
                                          u32x4 *__restrict__ Bnext,
                                          __amdgpu_buffer_rsrc_t arsrc, const uint32_t (&aoff)[16],
                                          const u32x4 &wc, const AbsRaw &ac, u32x4 &wn_, AbsRaw &an_,
                                          int64_t t, int64_t nsteps, int jl, int grp) {
  const int64_t t1 = (t + 1 < nsteps) ? t + 1 : nsteps - 1;
  const int64_t t2 = (t + 2 < nsteps) ? t + 2 : nsteps - 1;
  const uint32_t words[4] = {wc.x, wc.y, wc.z, wc.w};
  const float ta = prod.table_absmax(ac);
  Lut16 lut;
  WordLookup wl;
  uint32_t wout[2][4];
  // Fragment-read pair p of sub-step s into buffer n.
  auto read_pair = [&](int s, int p, int n) {
    const int u = 2 * s + grp;
    if (p < 2) {
      a[n][2 * p] = Acur[lds_unit(64 * p + jl, u)];
      a[n][2 * p + 1] = Acur[lds_unit(64 * p + 32 + jl, u)];
    } else {
      b[n][2 * (p - 2)] = Bcur[lds_unit_b(64 * (p - 2) + jl, u)];
      b[n][2 * (p - 2) + 1] = Bcur[lds_unit_b(64 * (p - 2) + 32 + jl, u)];
    }
  };
  auto dma = [&](int d) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void_t *)(Anext_wave + d * 64), 16,
                                             (int)aoff[d], (int)(t1 * (kStep * 2)), 0, 0);
  };
  auto word_stage = [&](int k, int stage) {
    if (stage == 0) word_select(words[k], wl);
    if (stage == 1) word_even(lut, wl);
    if (stage == 2) word_odd(lut, wl);
    if (stage == 3) {
      Producer::merge(wl, wout[k & 1]);
      if (Producer::kStoreParts == 1) prod.store(Bnext, wout[k & 1], k, 0);
    }
  };
  auto store_part = [&](int k, int p) {
    if (Producer::kStoreParts > 1) prod.store(Bnext, wout[k & 1], k, p);
  };
  // Previous step's tail, then this step's sub-step 0 fragments.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[3][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, b[1][i]), __builtin_bit_cast(bf16x8, a[1][3]), acc[3][i], 0,
        0, 0);
    read_pair(0, i, 0);
    if (i == 3) prod.load(g, t2, wn_, an_);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int n = (s + 1) & 1;
#pragma unroll
    for (int i = 0; i < ((s == 3) ? 12 : 16); ++i) {
      const int mt = i >> 2, nt = i & 3;
      acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
          __builtin_bit_cast(bf16x8, b[s & 1][nt]), __builtin_bit_cast(bf16x8, a[s & 1][mt]),
          acc[mt][nt], 0, 0, 0);
      const int q = i & 3;  // position inside the slot group
      if (s < 3 && i < 4) read_pair(s + 1, q, n);
      if (Producer::kStoreParts == 1) {
        if (s < 2 && i >= 8) dma(8 * s + (i - 8));
      } else {
        if (s < 2 && i < 4) dma(8 * s + q);
        if (s < 2 && i >= 12) dma(8 * s + 4 + q);
      }
      if (s == 0 && i >= 4 && i < 8) make_lut_quarter<false>(ta, q, lut);
      if (s == 0 && i >= 8 && i < 12) word_stage(0, q);
      if (s > 0 && i >= 4 && i < 8) word_stage(s, q);
      if (s > 0 && i >= 8 && i < 12) store_part(s - 1 + (s == 3 ? 1 : 0), q);
      if (s == 3 && i < 4) store_part(2, q);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// The last step's tail (see gemm_step).
__device__ __forceinline__ void gemm_tail(floatx16 (&acc)[4][4], const u32x4 (&a)[2][4],
                                          const u32x4 (&b)[2][4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc[3][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, b[1][i]), __builtin_bit_cast(bf16x8, a[1][3]), acc[3][i], 0,
        0, 0);
}

template <class Producer>
__global__ void __launch_bounds__(kGemmThreads, 1) nf4_gemm_kernel(const GemmArgs g) {
  int tm, to;
  map_tile(g.tiles_m, g.tiles_o, tm, to);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int jl = lane & 31;
  const int grp = lane >> 5;
  const int64_t m0 = (int64_t)tm * kTileM + wave * 128;
  const int64_t o0 = (int64_t)to * kTileO;
  const int64_t nsteps = g.R / kStep;

  // Direct-to-LDS activation loads: instruction i writes rows 8i..8i+7 of the
  // wave's 128-row tile as 1 KB, lane p at LDS unit 64i + p, i.e. row
  // 8i + p/8, physical unit p%8, which holds logical unit (p%8) ^ (row%8)
  // (the swizzle of lds_unit).  aoff[i] is lane p's byte offset from the
  // wave's first (clamped) row at k = 0; rows beyond M are clamped.  The
  // loads go through a buffer resource based at that row, with the step's
  // k offset in a scalar register, so the loop spends no vector ALU work on
  // their addresses (check_gemm bounds every offset below 2^31).
  const int64_t mb = (m0 < g.M) ? m0 : g.M - 1;
  const char *abase = reinterpret_cast<const char *>(g.a + mb * g.lda);
  // Rows available to this wave from mb (at least 1, at most 128).
  const int64_t avail64 = g.M - mb;
  const int32_t avail = (int32_t)(avail64 > 128 ? 128 : avail64);
  const uint32_t lda2 = (uint32_t)(g.lda * 2);
  const int32_t skip = (int32_t)(m0 - mb);  // > 0 only when the whole wave is past M
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc((void *)abase, 0, 0x7fffffff, kBufferFlags);
  uint32_t aoff[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rr = 8 * i + (lane >> 3);
    int rel = rr + skip;
    if (rel > avail - 1) rel = avail - 1;
    const int u = (lane & 7) ^ (rr & 7);
    aoff[i] = (uint32_t)rel * lda2 + 16u * (uint32_t)u;
  }

  Producer prod;
  prod.init(g, o0);

  floatx16 acc[4][4];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][nt][v] = 0.0f;

  u32x4 *a0w = &g_lds_a[wave][0][0];
  u32x4 *a1w = &g_lds_a[wave][1][0];

  // Prologue: activation tile of step 0 (DMA), weight tile of step 0
  // (dequantized into b0), packed weights of step 1 in registers.
#pragma unroll
  for (int i = 0; i < 16; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void_t *)(a0w + i * 64), 16, (int)aoff[i],
                                             0, 0, 0);
  {
    u32x4 w0;
    AbsRaw s0;
    prod.load(g, 0, w0, s0);
    prod.store(g_lds_b[0], w0, s0);
  }
  u32x4 wc, wn;
  AbsRaw ac, an;
  prod.load(g, nsteps > 1 ? 1 : 0, wc, ac);
  __builtin_amdgcn_s_waitcnt(0);  // the DMA of step 0 has landed in LDS
  __syncthreads();

  // Fragment registers; the first step's tail multiplies zeros.
  u32x4 fa[2][4], fb[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    fa[1][i] = (u32x4){0u, 0u, 0u, 0u};
    fb[1][i] = (u32x4){0u, 0u, 0u, 0u};
  }

  // Two steps per iteration, even then odd buffers; the packed-weight
  // registers swap roles instead of being copied.  After each step the next
  // step's activation tile (direct-to-LDS) and weight tile are complete.
  // The last step's "next" work reads clamped (valid) addresses and fills
  // buffers nobody reads again.
#pragma unroll 1
  for (int64_t t = 0; t + 1 < nsteps; t += 2) {
    gemm_step<Producer>(g, prod, acc, fa, fb, a0w, a1w, g_lds_b[0], g_lds_b[1], arsrc, aoff, wc,
                        ac, wn, an, t, nsteps, jl, grp);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    gemm_step<Producer>(g, prod, acc, fa, fb, a1w, a0w, g_lds_b[1], g_lds_b[0], arsrc, aoff, wn,
                        an, wc, ac, t + 1, nsteps, jl, grp);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  if (nsteps & 1) {
    gemm_step<Producer>(g, prod, acc, fa, fb, a0w, a1w, g_lds_b[0], g_lds_b[1], arsrc, aoff, wc,
                        ac, wn, an, nsteps - 1, nsteps, jl, grp);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }
  gemm_tail(acc, fa, fb);

  // Epilogue: fp32 -> bf16 (RNE).  The MFMAs take the weight fragment as
  // their first operand, so each accumulator tile is the transposed output
  // block: lane l holds activation row m0 + 32mt + l%32 and output columns
  // o0 + 32nt + 8j + 4g + i (i = 0..3) in registers 4j + i.  Four adjacent
  // columns leave as one 8-byte store.
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(g.out) & 7) == 0) && ((g.ldo & 3) == 0);
  const int64_t cl = g.O - (o0 + 4 * grp);
  const int32_t clim = (int32_t)(cl < 0 ? 0 : (cl > (1 << 30) ? (1 << 30) : cl));
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int64_t m = m0 + 32 * mt + jl;
    if (m < g.M) {
      uint16_t *orow = g.out + m * g.ldo + o0 + 4 * grp;
#pragma unroll
      for (int nt = 0; nt < 4; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = 32 * nt + 8 * j;
          const uint32_t lo = pack_bf16x2(acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1]);
          const uint32_t hi = pack_bf16x2(acc[mt][nt][4 * j + 2], acc[mt][nt][4 * j + 3]);
          if (vec_ok && c + 4 <= clim) {
            *reinterpret_cast<u32x2 *>(orow + c) = (u32x2){lo, hi};
          } else {
            if (c < clim) orow[c] = (uint16_t)(lo & 0xffffu);
            if (c + 1 < clim) orow[c + 1] = (uint16_t)(lo >> 16);
            if (c + 2 < clim) orow[c + 2] = (uint16_t)(hi & 0xffffu);
            if (c + 3 < clim) orow[c + 3] = (uint16_t)(hi >> 16);
          }
        }
    }
  }
}

static AbsmaxRef absmax_of(const nf4s_tensor &t) {
  AbsmaxRef a;
  a.absmax = t.absmax;
  a.q = t.absmax_q;
  a.scale = t.absmax_scale;
  a.group_shift = t.dq_group > 0 ? group_shift(t.dq_group) : 0;
  return a;
}

// Shared argument checks of the two GEMM entry points.  W is [wn, wk].
static int32_t check_gemm(const uint16_t *act, const nf4s_tensor *w, int64_t m, int64_t wn,
                          int64_t wk, const uint16_t *out) {
  if (act == nullptr || out == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "activation or output is NULL");
  if (m < 0 || wn <= 0 || wk <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad GEMM shape m=%lld n=%lld k=%lld",
                (long long)m, (long long)wn, (long long)wk);
  const int32_t rc = validate_tensor(w, wn * wk);
  if (rc != NF4S_OK) return rc;
  if (w->block_size != 64)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "fused GEMM needs block_size 64, got %d",
                w->block_size);
  if (wk % 64 != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "fused GEMM needs k %% 64 == 0, got %lld",
                (long long)wk);
  if (!aligned(act, 16) || !aligned(w->packed, 16))
    return fail(NF4S_ERR_MISALIGNED, "activation and packed weights must be 16-byte aligned");
  if (!aligned(out, 2)) return fail(NF4S_ERR_MISALIGNED, "output must be 2-byte aligned");
  return NF4S_OK;
}

// The activation loads address a wave's 128 rows with 32-bit offsets.
static int32_t check_offsets(int64_t lda) {
  if (lda > (int64_t)1 << 22)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "activation row of %lld elements is too long",
                (long long)lda);
  return NF4S_OK;
}

template <class Producer>
static int32_t launch_gemm(const GemmArgs &g, hipStream_t s, const char *name) {
  const int64_t T = (int64_t)g.tiles_m * g.tiles_o;
  if (T == 0) return NF4S_OK;
  if (T > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
  hipLaunchKernelGGL(nf4_gemm_kernel<Producer>, dim3((uint32_t)T), dim3(kGemmThreads), 0, s, g);
  return check_launch(name);
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

int32_t nf4s_gemm_fwd(const uint16_t *x, const nf4s_tensor *w, int64_t m, int64_t n, int64_t k,
                      uint16_t *y, void *stream) {
  int32_t rc = check_gemm(x, w, m, n, k, y);
  if (rc == NF4S_OK) rc = check_offsets(k);
  if (rc != NF4S_OK) return rc;
  if (m == 0) return NF4S_OK;
  GemmArgs g{};
  g.a = x;
  g.lda = k;
  g.out = y;
  g.ldo = n;
  g.M = m;
  g.O = n;
  g.R = k;
  g.packed = w->packed;
  g.am = absmax_of(*w);
  g.wk = k;
  g.wn = n;
  g.tiles_m = (int32_t)((m + kTileM - 1) / kTileM);
  g.tiles_o = (int32_t)((n + kTileO - 1) / kTileO);
  if (w->absmax_q != nullptr)
    return launch_gemm<FwdProducer<true>>(g, as_stream(stream), "nf4_gemm_fwd");
  return launch_gemm<FwdProducer<false>>(g, as_stream(stream), "nf4_gemm_fwd");
}

int32_t nf4s_gemm_dgrad(const uint16_t *dy, const nf4s_tensor *w, int64_t m, int64_t n,
                        int64_t k, uint16_t *dx, void *stream) {
  int32_t rc = check_gemm(dy, w, m, n, k, dx);
  if (rc == NF4S_OK) rc = check_offsets(n);
  if (rc != NF4S_OK) return rc;
  if (n % 64 != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "dgrad needs n %% 64 == 0, got %lld", (long long)n);
  if (m == 0) return NF4S_OK;
  GemmArgs g{};
  g.a = dy;
  g.lda = n;
  g.out = dx;
  g.ldo = k;
  g.M = m;
  g.O = k;
  g.R = n;
  g.packed = w->packed;
  g.am = absmax_of(*w);
  g.wk = k;
  g.wn = n;
  g.tiles_m = (int32_t)((m + kTileM - 1) / kTileM);
  g.tiles_o = (int32_t)((k + kTileO - 1) / kTileO);
  if (w->absmax_q != nullptr)
    return launch_gemm<DgradProducer<true>>(g, as_stream(stream), "nf4_gemm_dgrad");
  return launch_gemm<DgradProducer<false>>(g, as_stream(stream), "nf4_gemm_dgrad");
}

}  // extern "C"
