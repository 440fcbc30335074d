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
#include <type_traits>

#include "abi_common.hpp"
#include "gemm_common.hpp"
#include "nf4_device.hpp"

namespace nf4s {

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
  int64_t k0;         // first reduction step (a split-K slice's start; else 0)
  int32_t tiles_m, tiles_o;
};

// LDS tile: 128 rows x 64 bf16 (128 B = 8 units of 16 B).  A 16-B access
// (ds_read_b128, ds_write_b128) is served 16 lanes at a time, 256 B over the
// 64 banks, and the lanes of one group cover 16 consecutive rows at one
// logical unit.  Unit u of row r lives at r*8 + (u ^ swz(r)), where swz(r)
// takes 8 distinct values over the even rows and over the odd rows of every
// aligned group of 16 (and over every aligned group of 8 rows), so each
// group of 16 lanes touches 16 distinct 16-B bank windows.
__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
__device__ __forceinline__ int lds_unit(int row, int u) { return row * 8 + (u ^ swz(row)); }

// Weight tile: the same swizzle XOR 2 * ((row / 32) % 4).  The extra term is
// constant over each aligned group of 16 rows, so fragment reads stay spread
// over the banks, and it spreads the dgrad producer's 16-bit stores (whose
// lanes cover output columns 32 apart) over all banks too.
__device__ __forceinline__ int lds_unit_b(int row, int u) {
  return row * 8 + (u ^ swz(row) ^ ((row >> 4) & 6));
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

// Producer interface used by the GEMM step (phase = step index mod kUnroll):
//   prologue_load / prologue_store   loads for steps 0 and 1; step 0's tile
//   issue_loads<phase>(g, t, nsteps) loads issued in step t for later steps
//   prepare<phase>()                 register work once those loads landed
//   word<phase>(k), table_absmax<phase>()
//                                    packed word k and absmax of step t+1,
//                                    the tile dequantized during step t
//   finish<phase>()                  end of step t
//   store<kPar, k, part>(lds, out)   writes the dequantized word k.
//
// Per-step loading (PerStepLoads): step t loads the packed words and raw
// absmax of step t+2 into register set t & 1; step t+1's tile comes from the
// other set, loaded a step earlier.
template <bool kDQ, class Derived>
struct PerStepLoads {
  static constexpr int kUnroll = 2;
  u32x4 w[2];
  AbsRaw a[2];
  u32x4 w0;  // step 0 (prologue)
  AbsRaw a0;
  __device__ __forceinline__ void prologue_load(const GemmArgs &g, int nsteps) {
    const Derived &d = static_cast<const Derived &>(*this);
    d.load_step(g, 0, w0, a0);
    d.load_step(g, nsteps > 1 ? 1 : 0, w[1], a[1]);
  }
  template <int kPhase>
  __device__ __forceinline__ void issue_loads(const GemmArgs &g, int t, int nsteps) {
    const int t2 = (t + 2 < nsteps) ? t + 2 : nsteps - 1;
    static_cast<const Derived &>(*this).load_step(g, t2, w[kPhase & 1], a[kPhase & 1]);
  }
  template <int kPhase>
  __device__ __forceinline__ void prepare() {}
  template <int kPhase>
  __device__ __forceinline__ void finish() {}
  template <int kPhase>
  __device__ __forceinline__ uint32_t word(int k) const {
    return w[(kPhase + 1) & 1][k];
  }
  template <int kPhase>
  __device__ __forceinline__ float table_absmax() const {
    return static_cast<const Derived &>(*this).masked(absmax_value<kDQ>(a[(kPhase + 1) & 1]));
  }
  __device__ __forceinline__ void prologue_store(u32x4 *lds) const {
    const Derived &d = static_cast<const Derived &>(*this);
    d.store_tile(lds, w0, d.masked(absmax_value<kDQ>(a0)));
  }
};

// The product table of a block shared by the two lanes that dequantize it
// (the two 32-element halves of one 64-element block): lane half h builds
// table entries 8h .. 8h+7 (8 products, 4 conversions, 4 byte-plane perms,
// half the work) and receives the other 8 from its partner by DPP.  Its table
// registers then hold (own entries, partner's entries): entries 0-7 first on
// an h = 0 lane, entries 8-15 first on an h = 1 lane.  The lookup picks the
// table half by bit 3 of the nibble, so an h = 1 lane flips bit 3 of every
// nibble of its packed words first (hmask): code c is looked up at c ^ 8,
// where that lane keeps it.  Each product still depends on (code, absmax)
// only, so every element keeps the reference's bits.
struct HalfTable {
  uint32_t hmask;  // 0x88888888 on an h = 1 lane, else 0
  float code[8];   // NF4 codes 8h .. 8h+7
  __device__ __forceinline__ void init_half(int h) {
    hmask = h ? 0x88888888u : 0u;
#pragma unroll
    for (int j = 0; j < 8; ++j) code[j] = h ? code_value(8 + j) : code_value(j);
  }
};

// Forward producer: thread -> (row n_local, half h), 32 consecutive k of one
// block; writes 4 swizzled 16-B units of its row.  Lanes 16j..16j+15 of a
// wave take 8 consecutive rows, lanes 16j..16j+7 their half 0 and lanes
// 16j+8..16j+15 their half 1, so the two lanes of a block are 8 apart in one
// 16-lane DPP row (row_ror:8 swaps them), and each 8-lane group of a
// ds_write_b128 (a 128-B bank window) covers 8 consecutive rows at one
// logical unit, 8 distinct physical units (no bank conflicts).  FwdStore
// holds that mapping and the stores; the two forward producers differ only
// in how the packed words and absmax reach the registers.
struct FwdStore : HalfTable {
  static constexpr bool kFwd = true;
  static constexpr int kDppPartner = 0x128;  // row_ror:8: lane ^ 8 within 16
  int row, h;
  __device__ __forceinline__ void init_row() {
    const int lane = threadIdx.x & 63;
    row = 32 * (threadIdx.x >> 6) + 16 * (lane >> 5) + 8 * ((lane >> 4) & 1) + (lane & 7);
    h = (lane >> 3) & 1;
    init_half(h);
  }
  __device__ __forceinline__ float masked(float a) const { return a; }
  // Writes the 8 dequantized elements of packed word k (natural order).
  template <int kPar, int k, int kPart>
  __device__ __forceinline__ void store(u32x4 *lds, const uint32_t out[4]) const {
    u32x4 v;
    v.x = out[0]; v.y = out[1]; v.z = out[2]; v.w = out[3];
    lds[lds_unit_b(row, 4 * h + k)] = v;
  }
  // Fragment j of sub-step s: tile rows 32j + jl, reduction unit 2s + grp.
  __device__ __forceinline__ void read_b(const u32x4 *Bcur, u32x4 &out, int s, int j, int jl,
                                         int grp) const {
    out = Bcur[lds_unit_b(32 * j + jl, 2 * s + grp)];
  }
  // Whole-tile store (prologue).
  __device__ __forceinline__ void store_tile(u32x4 *lds, const u32x4 &w, float am) const {
    const Lut16 lut = make_lut<false>(am);
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    static_for<0, 4>([&](auto K) {
      constexpr int k = decltype(K)::value;
      uint32_t o[4];
      WordLookup x;
      word_select(words[k], x);
      word_even(lut, x);
      word_odd(lut, x);
      word_merge(x, o);
      this->template store<0, k, 0>(lds, o);
    });
  }
};

// Forward producer with one load per step and thread (any k % 64 == 0, any
// block size 64 << s with k % block_size == 0: the block of absolute step t
// is t >> s, so a step never straddles two blocks and both lanes of a row's
// 64 elements share one block).
template <bool kDQ>
struct FwdProducer : FwdStore, PerStepLoads<kDQ, FwdProducer<kDQ>> {
  const uint8_t *ptr;   // packed bytes of (row, half) at step 0
  int64_t am_row;       // absmax block index of the row's first block
  int64_t k0;           // absolute step of step 0
  AbsmaxRef am;
  // Tile row r takes W row n0 + r (n0 = the tile's first output column).
  __device__ void init(const GemmArgs &g, int64_t n0, uint32_t b0_lds) {
    (void)b0_lds;
    init_row();
    int64_t n = n0 + row;
    if (n >= g.wn) n = g.wn - 1;  // ragged N: clamp (outputs are not stored)
    ptr = g.packed + n * (g.wk >> 1) + 16 * h + 32 * g.k0;
    am = g.am;
    am_row = n * (g.wk >> (6 + am.block_shift));
    k0 = g.k0;
  }
  __device__ __forceinline__ void load_step(const GemmArgs &g, int step, u32x4 &w,
                                            AbsRaw &a) const {
    (void)g;
    w = *reinterpret_cast<const u32x4 *>(ptr + (int64_t)step * 32);
    a = absmax_load<kDQ>(am, am_row + ((k0 + step) >> am.block_shift));
  }
};

// Forward producer with batched loads (k % 256 == 0, 4-step unroll).  A
// thread's per-step data (16 B of packed nibbles, one absmax) sits in a
// different cache line for each of the wave's 32 rows, and the activation
// stream evicts those lines before the next step comes back to them.  So:
//  * packed nibbles are loaded two steps at a time: instruction X covers the
//    wave's rows 0-15 and instruction Y rows 16-31, 64 contiguous bytes per
//    row (lane l: row 8 ((l / 16) % 2) + l % 8, 16-B chunk c = 2 (l / 32) +
//    (l / 8) % 2 = (step 2p + c / 2, half c % 2)).  v_permlane32_swap then
//    exchanges X's upper 32 lanes with Y's lower 32: X holds step 2p and Y
//    step 2p+1, both in the thread -> (row, half) layout of FwdStore.  Half
//    the cache lines per step.
//  * absmax is loaded four steps at a time: one dword of double-quant codes
//    (or one float4 of fp32 absmax) plus one scale per thread.  The four
//    blocks lie in one scale group (dq_group >= 4, and 4 | blocks per row).
// Registers: pair set 0 is loaded in phase 0 (steps t+2, t+3), pair set 1 in
// phase 2; the absmax of group t/4 + 1 in phase 0.
template <bool kDQ>
struct FwdBatchProducer : FwdStore {
  static constexpr int kUnroll = 4;
  const uint8_t *pkx, *pky;  // pair loads of instructions X and Y at pair 0
  int64_t am_idx;            // absmax block index of (row) at step 0
  int npairs, ngroups;
  u32x4 X[2], Y[2];
  typedef typename std::conditional<kDQ, u32x2, u32x4>::type Group;
  Group cur, nxt;  // kDQ: {codes of 4 blocks, scale bits}; else 4 fp32 absmax
  AbsmaxRef am;

  // Tile row r takes W row n0 + r (n0 = the tile's first output column).
  __device__ void init(const GemmArgs &g, int64_t n0, uint32_t b0_lds) {
    (void)b0_lds;
    init_row();
    const int lane = threadIdx.x & 63;
    int64_t n = n0 + row;
    if (n >= g.wn) n = g.wn - 1;
    am_idx = n * (g.wk >> 6) + g.k0;  // absolute block: scale groups stay aligned
    am = g.am;
    int64_t nx = n0 + 32 * (threadIdx.x >> 6) + 8 * ((lane >> 4) & 1) + (lane & 7);
    int64_t ny = nx + 16;
    if (nx >= g.wn) nx = g.wn - 1;
    if (ny >= g.wn) ny = g.wn - 1;
    const int chunk = 2 * (lane >> 5) + ((lane >> 3) & 1);
    pkx = g.packed + nx * (g.wk >> 1) + 16 * chunk + 32 * g.k0;
    pky = g.packed + ny * (g.wk >> 1) + 16 * chunk + 32 * g.k0;
    npairs = (int)(g.R >> 7);
    ngroups = (int)(g.R >> 8);
  }
  __device__ __forceinline__ void load_pair(int p, u32x4 &x, u32x4 &y) const {
    x = *reinterpret_cast<const u32x4 *>(pkx + (int64_t)p * 64);
    y = *reinterpret_cast<const u32x4 *>(pky + (int64_t)p * 64);
  }
  __device__ __forceinline__ void load_group(const GemmArgs &g, int gi, Group &v) const {
    (void)g;
    const int64_t blk = am_idx + 4 * (int64_t)gi;
    if constexpr (kDQ) {
      v.x = *reinterpret_cast<const uint32_t *>(am.q + blk);
      v.y = __builtin_bit_cast(uint32_t, am.scale[blk >> am.group_shift]);
    } else {
      v = *reinterpret_cast<const u32x4 *>(am.absmax + blk);
    }
  }
  // The vector elements are copied to scalars before the bit casts:
  // __builtin_bit_cast of an ext_vector element expression reads element 0.
  template <int b>
  static __device__ __forceinline__ float group_absmax(const Group &v) {
    if constexpr (kDQ) {
      const uint32_t q = v.x, s = v.y;
      return (float)((q >> (8 * b)) & 0xffu) * __builtin_bit_cast(float, s);
    } else {
      const uint32_t a = v[b];
      return __builtin_bit_cast(float, a);
    }
  }
  static __device__ __forceinline__ void swap(u32x4 &x, u32x4 &y) {
    static_for<0, 4>([&](auto I) {
      constexpr int i = decltype(I)::value;
      const auto r = __builtin_amdgcn_permlane32_swap(x[i], y[i], false, false);
      x[i] = r[0];
      y[i] = r[1];
    });
  }
  __device__ __forceinline__ void prologue_load(const GemmArgs &g, int nsteps) {
    (void)nsteps;
    load_pair(0, X[1], Y[1]);
    load_group(g, 0, cur);
  }
  __device__ __forceinline__ void prologue_store(u32x4 *lds) {
    swap(X[1], Y[1]);
    store_tile(lds, X[1], group_absmax<0>(cur));
  }
  template <int kPhase>
  __device__ __forceinline__ void issue_loads(const GemmArgs &g, int t, int nsteps) {
    (void)nsteps;
    if constexpr (kPhase == 0 || kPhase == 2) {
      int p = (t + 2) >> 1;
      if (p > npairs - 1) p = npairs - 1;  // look-ahead past the end: unused
      load_pair(p, X[kPhase >> 1], Y[kPhase >> 1]);
    }
    if constexpr (kPhase == 0) {
      int gi = (t >> 2) + 1;
      if (gi > ngroups - 1) gi = ngroups - 1;
      load_group(g, gi, nxt);
    }
  }
  template <int kPhase>
  __device__ __forceinline__ void prepare() {
    if constexpr (kPhase == 1) swap(X[0], Y[0]);
    if constexpr (kPhase == 3) swap(X[1], Y[1]);
  }
  template <int kPhase>
  __device__ __forceinline__ uint32_t word(int k) const {
    if constexpr (kPhase == 0) return Y[1][k];
    else if constexpr (kPhase == 1) return X[0][k];
    else if constexpr (kPhase == 2) return Y[0][k];
    else return X[1][k];
  }
  template <int kPhase>
  __device__ __forceinline__ float table_absmax() const {
    if constexpr (kPhase == 3) return group_absmax<0>(nxt);
    else return group_absmax<kPhase + 1>(cur);
  }
  template <int kPhase>
  __device__ __forceinline__ void finish() {
    if constexpr (kPhase == 3) cur = nxt;
  }
};

// Dgrad producer: the step covers W rows n0..n0+63 (the reduction) and W
// columns o0..o0+127 (the output).  Thread -> (W row r = tid/4, quarter
// q = tid%4): 32 consecutive columns of one block, dequantized as 4 words of
// 8 elements and written as 4 16-B units.  The LDS tile keeps W's layout:
// row r (256 B) holds the tile's 128 columns; logical unit u (columns
// 8u..8u+7) sits at physical unit (u ^ 2 (u / 8)) ^ 5 (r % 4).
//
// The MFMA fragment of output column o holds 8 consecutive reduction values,
// a column of this tile.  ds_read_b64_tr_b16 transposes 4 x 4 blocks of
// 16-bit values within each 16-lane group: lane i of the group receives
// element i % 4 of the 8 bytes addressed by lane 4e + i / 4, e = 0..3.  So
// when lane 4e + c addresses row e, columns 4c..4c+3 of a 16-column strip,
// lane i receives column i of rows 0..3, and two such reads (rows 0-3, 4-7)
// make the fragment.
//
// Banks: a ds_write_b128 is served 8 lanes at a time over a 128-B window
// (bank group = address / 16 mod 8; measured with an LDS probe: the plain
// XOR layout u ^ 5 (r % 4) cost 8 conflict cycles per store, this one none).
// Its 8 lanes are rows r, r + 1 (c = r % 4 and c + 1) at quarters 0..3 and
// one word k: physical units 4 (q ^ c) + ((k ^ 2 (q / 2)) ^ c), whose values
// mod 8 are {k', 4 + k', k' ^ 2, 4 + (k' ^ 2)} for k' = k ^ c, disjoint for
// the two rows.  A 32-lane half of a transposed read covers c = 0..3 at
// logical units 4j..4j+3 (fragment j), physical units
// 4 (j ^ c) + ((u % 4 ^ 2 (j / 2)) ^ c), 16 distinct.
// DgradStore holds the thread mapping, the LDS stores and the transposed
// fragment reads; the two input-gradient producers differ only in how the
// packed words and absmax reach the registers.
struct DgradStore : HalfTable {
  static constexpr bool kFwd = false;
  static constexpr int kDppPartner = 0xB1;   // quad_perm [1,0,3,2]: lane ^ 1
  uint32_t valid_mask;  // all ones when the thread's columns exist
  int sidx[4];          // LDS unit of the thread's word k
  uint32_t roff[4];     // byte offset of the lane's read of fragment j (rows 0-3 of sub-step 0)
  // Quarters 2b and 2b + 1 of a row are the two halves of its block b.
  __device__ void init_layout(const GemmArgs &g, int64_t o0) {
    const int r = threadIdx.x >> 2, q = threadIdx.x & 3, c = r & 3;
    init_half(q & 1);
#pragma unroll
    for (int k = 0; k < 4; ++k) sidx[k] = 16 * r + 4 * (q ^ c) + ((k ^ (2 * (q >> 1))) ^ c);
    const int lane = threadIdx.x & 63, l16 = lane & 15, cr = l16 >> 2;
    const int ub = 2 * ((lane >> 4) & 1) + ((l16 >> 1) & 1);  // unit within the fragment's 4
#pragma unroll
    for (int j = 0; j < 4; ++j)
      roff[j] = (uint32_t)(256 * (8 * (lane >> 5) + cr) +
                           16 * (4 * (j ^ cr) + ((ub ^ (2 * (j >> 1))) ^ cr)) + 8 * (l16 & 1));
    valid_mask = (o0 + 32 * q < g.wk) ? 0xffffffffu : 0u;
  }
  // Columns beyond k read column 0's bytes and are zeroed via the absmax.
  __device__ __forceinline__ float masked(float a) const {
    return __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, a) & valid_mask);
  }
  // Writes the 8 dequantized elements of packed word k (natural order).
  template <int kPar, int k, int kPart>
  __device__ __forceinline__ void store(u32x4 *lds, const uint32_t out[4]) const {
    u32x4 v;
    v.x = out[0]; v.y = out[1]; v.z = out[2]; v.w = out[3];
    lds[sidx[k]] = v;
  }
  // Fragment j of sub-step s: output columns 32j + lane % 32, reduction rows
  // 16s + 8(lane / 32) + 0..7.
  __device__ __forceinline__ void read_b(const u32x4 *Bcur, u32x4 &out, int s, int j, int jl,
                                         int grp) const {
    (void)jl;
    (void)grp;
    typedef __attribute__((address_space(3))) char lds_char_t;
    typedef __attribute__((address_space(3))) v4i16 lds_v4i16_t;
    lds_char_t *base = (lds_char_t *)const_cast<u32x4 *>(Bcur) + roff[j] + 4096 * s;
    const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)base);
    const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_t *)(base + 1024));
    const u32x2 l2 = __builtin_bit_cast(u32x2, lo), h2 = __builtin_bit_cast(u32x2, hi);
    out = (u32x4){l2.x, l2.y, h2.x, h2.y};
  }
  __device__ __forceinline__ void store_tile(u32x4 *lds, const u32x4 &w, float am) const {
    const Lut16 lut = make_lut<false>(am);
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    static_for<0, 4>([&](auto K) {
      constexpr int k = decltype(K)::value;
      uint32_t o[4];
      WordLookup x;
      word_select(words[k], x);
      word_even(lut, x);
      word_odd(lut, x);
      word_merge(x, o);
      this->template store<0, k, 0>(lds, o);
    });
  }
};

// Input-gradient producer with one packed load, one absmax code and one
// scale load per step and thread (any n % 64 == 0, k % 64 == 0).
// (Any block size 64 << s with k % block_size == 0: a row's blocks are
// block_size columns wide, and the two quarters of a 64-column half share a
// block.)
template <bool kDQ>
struct DgradProducer : DgradStore, PerStepLoads<kDQ, DgradProducer<kDQ>> {
  const uint8_t *ptr;
  int64_t am_idx;
  int64_t am_stride;  // blocks per 64 W rows
  AbsmaxRef am;
  __device__ void init(const GemmArgs &g, int64_t o0, uint32_t b0_lds) {
    (void)b0_lds;
    init_layout(g, o0);
    const int r = threadIdx.x >> 2, q = threadIdx.x & 3;
    const int64_t col = o0 + 32 * q;
    const int64_t cc = col < g.wk ? col : 0;
    const int64_t row = r + 64 * g.k0;  // a split-K slice starts at W row 64 k0
    ptr = g.packed + row * (g.wk >> 1) + (cc >> 1);
    am = g.am;
    const int bs = 6 + am.block_shift;  // log2(block_size)
    am_idx = row * (g.wk >> bs) + (cc >> bs);  // absolute block: scale groups stay aligned
    am_stride = 64 * (g.wk >> bs);
  }
  __device__ __forceinline__ void load_step(const GemmArgs &g, int step, u32x4 &w,
                                            AbsRaw &a) const {
    // Step s covers W rows 64s .. 64s+63.
    w = *reinterpret_cast<const u32x4 *>(ptr + (int64_t)step * 64 * (g.wk >> 1));
    a = absmax_load<kDQ>(am, am_idx + (int64_t)step * am_stride);
  }
};

// Input-gradient producer with batched absmax loads (k % 128 == 0, n % 256
// == 0, dq_group >= 2; a 4-step unroll).  A step's absmax is one value per
// (W row, block), and the thread's blocks of consecutive steps lie 64 rows
// apart, in different cache lines.  So the four threads of a row (quarters
// q = 0..3) load the absmax of four different steps: thread (r, q) loads,
// for step 4g + q, the two blocks' double-quant codes of row r (2 bytes) and
// their scale (or the two fp32 absmax), one group of four steps ahead.  In
// step t the absmax of step t + 1 then comes from quad lane (t + 1) % 4 by a
// DPP broadcast, and the thread keeps its own block's byte.  Two small loads
// per four steps instead of eight.  The packed words keep the per-step loads
// (a step's 16 bytes per thread come from one row, the next step's from a
// row 64 further down).
template <bool kDQ>
struct DgradBatchProducer : DgradStore {
  static constexpr int kUnroll = 4;
  const uint8_t *ptr;       // packed bytes of (row r, quarter q) at step 0
  int64_t pstride;          // packed bytes per step (64 W rows)
  int64_t gblk;             // absmax block (row r + 64q, blocks b0, b0 + 1) of group 0
  int64_t gstride;          // blocks per group of 4 steps (256 W rows)
  int ngroups;
  uint32_t shift;           // 8 * (q >> 1): the thread's block within the pair
  AbsmaxRef am;
  u32x4 w[2];
  u32x4 w0;
  u32x2 cur, nxt;           // kDQ: {code pair, scale bits}; else {absmax b0, absmax b0 + 1}
  __device__ void init(const GemmArgs &g, int64_t o0, uint32_t b0_lds) {
    (void)b0_lds;
    init_layout(g, o0);
    const int r = threadIdx.x >> 2, q = threadIdx.x & 3;
    const int64_t row = r + 64 * g.k0;  // a split-K slice starts at W row 64 k0
    ptr = g.packed + row * (g.wk >> 1) + ((o0 + 32 * q) >> 1);
    pstride = 64 * (g.wk >> 1);
    gblk = (row + 64 * q) * (g.wk >> 6) + (o0 >> 6);  // absolute block
    gstride = 256 * (g.wk >> 6);
    ngroups = (int)(g.R >> 8);
    shift = 8u * (uint32_t)(q >> 1);
    am = g.am;
  }
  __device__ __forceinline__ void load_group(int gi, u32x2 &v) const {
    const int64_t blk = gblk + (int64_t)gi * gstride;
    if constexpr (kDQ) {
      v.x = *reinterpret_cast<const uint16_t *>(am.q + blk);
      v.y = __builtin_bit_cast(uint32_t, am.scale[blk >> am.group_shift]);
    } else {
      v = *reinterpret_cast<const u32x2 *>(am.absmax + blk);
    }
  }
  // Element i (step 4g + i) of a group, from quad lane i.  The vector
  // elements are copied to scalars first (see FwdBatchProducer).
  template <int i>
  __device__ __forceinline__ float group_absmax(const u32x2 &v) const {
    const uint32_t x = v.x, y = v.y;
    const uint32_t bx = (uint32_t)__builtin_amdgcn_mov_dpp((int)x, i * 0x55, 0xf, 0xf, false);
    const uint32_t by = (uint32_t)__builtin_amdgcn_mov_dpp((int)y, i * 0x55, 0xf, 0xf, false);
    if constexpr (kDQ) {
      return (float)((bx >> shift) & 0xffu) * __builtin_bit_cast(float, by);
    } else {
      return __builtin_bit_cast(float, shift != 0u ? by : bx);
    }
  }
  __device__ __forceinline__ void load_words(int step, u32x4 &v) const {
    v = *reinterpret_cast<const u32x4 *>(ptr + (int64_t)step * pstride);
  }
  __device__ __forceinline__ void prologue_load(const GemmArgs &g, int nsteps) {
    (void)g;
    load_words(0, w0);
    load_words(nsteps > 1 ? 1 : 0, w[1]);
    load_group(0, cur);
  }
  __device__ __forceinline__ void prologue_store(u32x4 *lds) const {
    store_tile(lds, w0, masked(group_absmax<0>(cur)));
  }
  template <int kPhase>
  __device__ __forceinline__ void issue_loads(const GemmArgs &g, int t, int nsteps) {
    (void)g;
    const int t2 = (t + 2 < nsteps) ? t + 2 : nsteps - 1;
    load_words(t2, w[kPhase & 1]);
    if constexpr (kPhase == 0) {
      int gi = (t >> 2) + 1;
      if (gi > ngroups - 1) gi = ngroups - 1;  // look-ahead past the end: unused
      load_group(gi, nxt);
    }
  }
  template <int kPhase>
  __device__ __forceinline__ void prepare() {}
  template <int kPhase>
  __device__ __forceinline__ uint32_t word(int k) const {
    return w[(kPhase + 1) & 1][k];
  }
  template <int kPhase>
  __device__ __forceinline__ float table_absmax() const {
    if constexpr (kPhase == 3) return masked(group_absmax<0>(nxt));
    else return masked(group_absmax<kPhase + 1>(cur));
  }
  template <int kPhase>
  __device__ __forceinline__ void finish() {
    if constexpr (kPhase == 3) cur = nxt;
  }
};

// LDS: two activation buffers per wave (128 rows x 128 B = 16 KB each, a
// wave's pair adjacent) and two weight tiles (16 KB each): 160 KB, the gfx950
// maximum.  With the buffers of a pair 16 KB apart, the main loop (unrolled
// by two steps) addresses both through the LDS instructions' immediate
// offsets from loop-invariant lane addresses.
__shared__ u32x4 g_lds_a[4][2][1024];
__shared__ u32x4 g_lds_b[2][1024];

// Fragment read k (0..7) of sub-step s into register buffer n, in the order
// the sub-step's first MFMAs consume them: A0, B0, B1, B2, B3, A1, A2, A3.
// Fragment j of A holds rows 32j + jl of the activation tile; fragment j of
// B output columns 32j + jl of the weight tile (the producer's read_b).
template <class Producer>
__device__ __forceinline__ void read_frag(const Producer &prod, const u32x4 *__restrict__ Acur,
                                          const u32x4 *__restrict__ Bcur, u32x4 (&a)[2][4],
                                          u32x4 (&b)[2][4], int s, int k, int n, int jl, int grp) {
  if (k == 0 || k >= 5) {
    const int j = (k == 0) ? 0 : k - 4;
    a[n][j] = Acur[lds_unit(32 * j + jl, 2 * s + grp)];
  } else {
    prod.read_b(Bcur, b[n][k - 1], s, k - 1, jl, grp);
  }
}

// The per-step slot plan.  Slot n = 16 s + i follows MFMA i of sub-step s;
// sub-step 3 has 8 slots before the barrier, so a step has 56.  Job kinds:
//   R  two fragment reads of the next sub-step (slots 0-3 of sub-steps 0-2);
//      'n' is R plus an N job
//   M  one quarter of this lane's half of the product table (2 products,
//      1 conversion; the second and fourth also form the half-quarter's low /
//      high byte words)
//   D  the partner lane's half of the table, 4 DPP moves (after the 4 M jobs
//      and before the first lookup stage that reads the table)
//   W  one lookup stage of a packed word (NatLookup), in order: selectors,
//      plane controls, elements 0-3, elements 4-7, the bf16 pairs, the
//      16-B store
//   N  one activation DMA of the NEXT step's tile, rows 64-127, into the
//      other buffer
//   A  one activation DMA of the step after next (t+2), rows 0-63, into the
//      current buffer once this wave's reads of it have returned
//   .  the MFMA alone
// Each slot holds about the issue time of one MFMA (32 cycles), and an MFMA
// hides about 5 independent VALU instructions: the 8 products of this lane's
// half of the table go in 4 slots of 3-5 instructions.  The last weight-tile store (word 3's W
// stage 5) sits at slot 44, 11 slots before the barrier, whose lgkmcnt(0)
// must see it complete; the A jobs follow in the last slots, after a wait
// for this wave's fragment reads only (the LDS queue is in order, so the
// wait exempts the stores issued after the last R slot).  N jobs go early:
// the barrier exempts only the 8 A jobs.
// On MI355X this plan measured +1.3 % (70B gate forward) to +3 % (70B q
// input gradient) over one that stored the last word two slots before the
// barrier; the 16 DMAs all in the second half of the step (16 exempt at the
// barrier) measured 5-9 % slower, and the N jobs right after the barrier
// 3-4 % slower for the input gradient.  The input-gradient plan is the same:
// its B fragment reads (two transposed 8-byte reads each) sit in the same R
// slots.
constexpr int kDmaInFlight = 8;
constexpr char kPlanFwd[57] =
    "RnRnMMNMMNDWWWNN"
    "RnRnWWWWWWWWWWWW"
    "RRRRWWWWWWWWWA.A"
    ".AAAAAA.";
constexpr const char *kPlanDgrad = kPlanFwd;
// Number of jobs of kind c before slot n ('n' counts as N).
constexpr int plan_index(const char *plan, int n, char c) {
  int k = 0;
  for (int i = 0; i < n; ++i) k += (plan[i] == c) || (c == 'N' && plan[i] == 'n');
  return k;
}
// Weight-tile stores (W stage 5) issued after the plan's last R slot before
// slot n: the LDS operations a wait for the fragment reads may leave pending.
constexpr int stores_after_reads(const char *plan, int n) {
  int last_r = -1;
  for (int i = 0; i < n; ++i)
    if (plan[i] == 'R' || plan[i] == 'n') last_r = i;
  int stores = 0, j = 0;
  for (int i = 0; i < n; ++i)
    if (plan[i] == 'W') {
      if (i > last_r && j % 6 == 5) ++stores;
      ++j;
    }
  return stores;
}
// Shape of a plan: 56 slots; R/n at slots 0-3 of sub-steps 0-2; 8 N, 8 A, 24
// W, 4 M and 1 D jobs; the D job after the 4 M jobs and two slots after the
// last (a DPP read of a register the previous VALU wrote needs wait states);
// the product table complete before the first lookup stage that reads it (W
// stage 2 of word 0).
constexpr bool plan_ok(const char *plan) {
  int r = 0, w = 0;
  for (int i = 0; i < 56; ++i) {
    const bool rs = plan[i] == 'R' || plan[i] == 'n';
    if (rs != (i < 48 && i % 16 < 4)) return false;
    r += rs;
    if (plan[i] == 'D' && (plan_index(plan, i, 'M') != 4 || plan[i - 1] == 'M')) return false;
    if (plan[i] == 'W' && w++ == 2 && plan_index(plan, i, 'D') != 1) return false;
  }
  return plan[56] == 0 && r == 12 && plan_index(plan, 56, 'N') == 8 &&
         plan_index(plan, 56, 'A') == 8 && w == 24 && plan_index(plan, 56, 'M') == 4 &&
         plan_index(plan, 56, 'D') == 1;
}
static_assert(plan_ok(kPlanFwd), "forward slot plan");
static_assert(plan_ok(kPlanDgrad), "input-gradient slot plan");

// One 64-deep reduction step t: 4 sub-steps of 16 MFMAs over the activation
// tile in Acur (this wave's 128 rows) and the weight tile in Bcur.  Alongside
// the MFMAs it reads the next sub-step's fragments, dequantizes step t+1's
// packed weights (loaded by the producer in an earlier step) into Bnext,
// issues the producer's loads for later steps and moves activation rows into
// LDS with direct-to-LDS loads (1 KB = 8 whole 128-B rows per instruction):
// rows 64-127 of step t+1 into Aoth (read last in step t-1) and rows 0-63 of
// step t+2 into Acur after this wave's last reads of it.  Every DMA has at
// least a sub-step to land before the barrier that precedes its reads, and
// the barrier waits for all but the kDmaInFlight (8) most recent
// vector-memory operations.
// A wave issues in order, so other work only overlaps the matrix pipe when
// it sits between MFMAs; a sched_barrier fence after every slot keeps the
// plan's order.  (Empty asm statements that pinned each stage's inputs to
// its slot cost a hazard s_nop each and a register copy per table quarter,
// 40 nops and 11 moves per step; without them the stages stay in their
// slots and the step measured 0.4-1.3 % faster.)
//
// The step's barrier comes after MFMA 7 of sub-step 3.  The last 8 MFMAs
// (a[1][2..3] x b[1][0..3], operands already in registers) open the NEXT
// call, after the barrier, each followed by one fragment read of the new
// step's sub-step 0.  The first call runs them on zero operands.
template <class Producer, int kPhase>
__device__ __forceinline__ void gemm_step(const GemmArgs &g, Producer &prod,
                                          floatx16 (&acc)[4][4], u32x4 (&a)[2][4],
                                          u32x4 (&b)[2][4], u32x4 *Acur, u32x4 *Aoth,
                                          const u32x4 *Bcur, u32x4 *Bnext,
                                          __amdgpu_buffer_rsrc_t arsrc, const uint32_t (&aoff)[16],
                                          int t, int nsteps, int jl, int grp) {
  constexpr int kPar = 1 - (kPhase & 1);
  constexpr bool kFwd = Producer::kFwd;
  constexpr int kWordStages = 6;
  const int t1 = (t + 1 < nsteps) ? t + 1 : nsteps - 1;
  const int t2 = (t + 2 < nsteps) ? t + 2 : nsteps - 1;
  Lut16 lut;
  uint32_t lutd[2];
  uint32_t own[4];  // this lane's half: low / high byte words of its 2 quarters
  NatLookup wl;
  uint32_t wp[4][4];  // dequantized elements of each packed word, memory order
  float ta = 0.0f;
  auto dma = [&](u32x4 *dst, int d, int step) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void_t *)(dst + d * 64), 16,
                                             (int)aoff[d], (int)(step * (kStep * 2)), 0, 0);
  };

  // Previous step's last 8 MFMAs, then this step's sub-step 0 fragments.
  static_for<0, 8>([&](auto I) {
    constexpr int i = decltype(I)::value;
    constexpr int mt = 2 + (i >> 2), nt = i & 3;
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, b[1][nt]), __builtin_bit_cast(bf16x8, a[1][mt]),
        acc[mt][nt], 0, 0, 0);
    read_frag(prod, Acur, Bcur, a, b, 0, i, 0, jl, grp);
    if constexpr (i == 3) prod.template issue_loads<kPhase>(g, t, nsteps);
    if constexpr (i == 5) prod.template prepare<kPhase>();
    if constexpr (i == 6) ta = prod.template table_absmax<kPhase>();
    __builtin_amdgcn_sched_barrier(0);
  });
  static_for<0, 56>([&](auto N) {
    constexpr int n = decltype(N)::value;
    constexpr int s = n / 16, i = n % 16;
    constexpr int mt = i >> 2, nt = i & 3;
    constexpr char kind = kFwd ? kPlanFwd[n] : kPlanDgrad[n];
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, b[s & 1][nt]), __builtin_bit_cast(bf16x8, a[s & 1][mt]),
        acc[mt][nt], 0, 0, 0);
    if constexpr (kind == 'R' || kind == 'n') {
      read_frag(prod, Acur, Bcur, a, b, s + 1, 2 * i, (s + 1) & 1, jl, grp);
      read_frag(prod, Acur, Bcur, a, b, s + 1, 2 * i + 1, (s + 1) & 1, jl, grp);
    }
    if constexpr (kind == 'N' || kind == 'n')
      dma(Aoth, 8 + plan_index(kFwd ? kPlanFwd : kPlanDgrad, n, 'N'), t1);
    if constexpr (kind == 'A') {
      constexpr const char *plan = kFwd ? kPlanFwd : kPlanDgrad;
      constexpr int d = plan_index(plan, n, 'A');
      // The wave's reads of Acur (sub-step 3's fragments) have returned;
      // weight-tile stores issued after them may still be pending.
      if constexpr (d == 0)
        __builtin_amdgcn_s_waitcnt(kWaitLgkm0 | (stores_after_reads(plan, n) << 8));
      dma(Acur, d, t2);
    }
    if constexpr (kind == 'M') {
      // Entries 2j and 2j+1 of this lane's half of the table.
      constexpr int j = plan_index(kFwd ? kPlanFwd : kPlanDgrad, n, 'M');
      const float p0 = fp32_rounded(prod.code[2 * j] * ta);
      const float p1 = fp32_rounded(prod.code[2 * j + 1] * ta);
      lutd[j & 1] = pack_bf16x2(p0, p1);
      if constexpr (j & 1) {
        own[2 * (j >> 1)] = perm(lutd[1], lutd[0], 0x06040200u);
        own[2 * (j >> 1) + 1] = perm(lutd[1], lutd[0], 0x07050301u);
      }
    }
    if constexpr (kind == 'D') {
      // (own half, partner's half): see HalfTable.
      static_for<0, 2>([&](auto Q) {
        constexpr int q = decltype(Q)::value;
        lut.lo[q] = own[2 * q];
        lut.hi[q] = own[2 * q + 1];
        lut.lo[2 + q] = (uint32_t)__builtin_amdgcn_mov_dpp((int)own[2 * q], Producer::kDppPartner,
                                                           0xf, 0xf, false);
        lut.hi[2 + q] = (uint32_t)__builtin_amdgcn_mov_dpp((int)own[2 * q + 1],
                                                           Producer::kDppPartner, 0xf, 0xf, false);
      });
    }
    if constexpr (kind == 'W') {
      constexpr int j = plan_index(kFwd ? kPlanFwd : kPlanDgrad, n, 'W');
      constexpr int k = j / kWordStages, stage = j % kWordStages;
      if constexpr (stage == 0) {
        nat_select(prod.template word<kPhase>(k) ^ prod.hmask, wl);
      } else if constexpr (stage == 1) {
        nat_controls(wl);
      } else if constexpr (stage == 2) {
        nat_planes_a(lut, wl);
      } else if constexpr (stage == 3) {
        nat_planes_b(lut, wl);
      } else if constexpr (stage == 4) {
        nat_merge(wl, wp[k]);
      } else {
        prod.template store<kPar, k, 0>(Bnext, wp[k]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  });
  step_barrier<kDmaInFlight>();
  prod.template finish<kPhase>();
}

// The last step's final 8 MFMAs (see gemm_step).
__device__ __forceinline__ void gemm_tail(floatx16 (&acc)[4][4], const u32x4 (&a)[2][4],
                                          const u32x4 (&b)[2][4]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int mt = 2 + (i >> 2), nt = i & 3;
    acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8, b[1][nt]), __builtin_bit_cast(bf16x8, a[1][mt]), acc[mt][nt],
        0, 0, 0);
  }
}

// Prologue, main loop and tail of the GEMM.  The LDS buffers come in as
// distinct __restrict__ pointers: the compiler then knows that the
// activation DMAs into one buffer never alias the fragment reads of the
// other, and waits (vmcnt) only for the DMAs whose buffer a read touches.
template <class Producer>
__device__ __forceinline__ void gemm_main(const GemmArgs &g, Producer &prod,
                                          floatx16 (&acc)[4][4], u32x4 *__restrict__ A0,
                                          u32x4 *__restrict__ A1, u32x4 *__restrict__ B0,
                                          u32x4 *__restrict__ B1, __amdgpu_buffer_rsrc_t arsrc,
                                          const uint32_t (&aoff)[16], int nsteps, int jl,
                                          int grp) {
  // Prologue: the producer's loads for steps 0 and 1, the activation tile of
  // step 0 and rows 0-63 of step 1 (DMA), then the weight tile of step 0
  // dequantized into B0.  The fences fix the order of issue, so that
  // vmcnt(kDmaInFlight) at the barrier means "all but step 1's 8 DMAs" to
  // the compiler as to the hardware.
  prod.prologue_load(g, nsteps);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < 16; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void_t *)(A0 + i * 64), 16,
                                             (int)aoff[i], 0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  const int step1 = (nsteps > 1) ? kStep * 2 : 0;
#pragma unroll
  for (int i = 0; i < kDmaInFlight; ++i)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, (lds_void_t *)(A1 + i * 64), 16,
                                             (int)aoff[i], step1, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
  prod.prologue_store(B0);
  step_barrier<kDmaInFlight>();

  // Fragment registers; the first step's head multiplies zeros.
  u32x4 fa[2][4], fb[2][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    fa[1][i] = (u32x4){0u, 0u, 0u, 0u};
    fb[1][i] = (u32x4){0u, 0u, 0u, 0u};
  }

  // kUnroll steps per iteration; even phases use the even buffers (A0, B0
  // read, B1 written), odd phases the odd ones, so no register or pointer is
  // copied between steps.  The last steps' look-ahead work reads clamped
  // (valid) addresses and fills buffers nobody reads again.  A producer
  // with kUnroll 4 needs nsteps % 4 == 0 (checked at launch); with kUnroll 2
  // an odd last step runs alone.
  constexpr int U = Producer::kUnroll;
  int t = 0;
#pragma unroll 1
  for (; t + U <= nsteps; t += U) {
    static_for<0, U>([&](auto P) {
      constexpr int p = decltype(P)::value;
      if constexpr ((p & 1) == 0)
        gemm_step<Producer, p>(g, prod, acc, fa, fb, A0, A1, B0, B1, arsrc, aoff, t + p, nsteps,
                               jl, grp);
      else
        gemm_step<Producer, p>(g, prod, acc, fa, fb, A1, A0, B1, B0, arsrc, aoff, t + p, nsteps,
                               jl, grp);
    });
  }
  if constexpr (U == 2) {
    if (t < nsteps)
      gemm_step<Producer, 0>(g, prod, acc, fa, fb, A0, A1, B0, B1, arsrc, aoff, t, nsteps, jl,
                             grp);
  }
  gemm_tail(acc, fa, fb);
  // No LDS DMA may still be in flight when the workgroup's LDS is released.
  __builtin_amdgcn_s_waitcnt(0);
}

// Up to kMaxGroups weights per launch.  Forward: the weights share the
// activation x and each has its own output (q/k/v, gate/up); the output
// tiles of all groups form one grid.  Input gradient: the groups are
// reduction segments of one output, dx = sum_i dy_i . W_i.
constexpr int kMaxGroups = 4;
struct GemmGroup {
  const uint16_t *a;   // input gradient: dy_i
  int64_t lda;
  uint16_t *out;       // forward: y_i
  int64_t ldo;
  const uint8_t *packed;
  AbsmaxRef am;
  int64_t wn;          // rows of W_i (its n)
  int32_t tiles_o;     // forward: output tiles of this group
};
struct GroupedArgs {
  GemmArgs base;       // shapes and the shared operand (x, or dx)
  GemmGroup grp[kMaxGroups];
  int32_t ngroups;
  int32_t tiles_o;     // forward: output tiles over all groups
  // Forward split-K tail: tiles [full_tiles, T) run as `splits` slices of
  // `split_steps` reduction steps each, whose fp32 partial tiles go to `ws`
  // (kPartialFloats per slice) and are summed by nf4_gemm_fixup_kernel.
  int32_t full_tiles;  // T when there is no split
  int32_t splits;
  int32_t split_steps;
  float *ws;
};

// One slice's partial tile: 256 threads x 256 accumulators, stored in the
// accumulator register order, thread-interleaved in 16-byte units, so that
// the fixup kernel's thread t reads back exactly thread t's values.
constexpr int64_t kPartialFloats = (int64_t)kGemmThreads * 256;

// Buffer resource and per-lane offsets of the wave's direct-to-LDS
// activation loads: instruction i writes rows 8i..8i+7 of the wave's 128-row
// tile as 1 KB, lane p at LDS unit 64i + p, i.e. row 8i + p/8, physical unit
// p%8, which holds logical unit (p%8) ^ swz(row) (the swizzle of lds_unit).
// aoff[i] is lane p's byte offset from the wave's first (clamped) row at
// k = 0; rows beyond M are clamped.  The loads go through a buffer resource
// based at that row, with the step's k offset in a scalar register, so the
// loop spends no vector ALU work on their addresses (check_offsets bounds
// every offset below 2^31).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t activation_setup(const GemmArgs &g, int64_t m0,
                                                                   int lane, uint32_t (&aoff)[16]) {
  const int64_t mb = (m0 < g.M) ? m0 : g.M - 1;
  const char *abase = reinterpret_cast<const char *>(g.a + mb * g.lda + kStep * g.k0);
  // Rows available to this wave from mb (at least 1, at most 128).
  const int64_t avail64 = g.M - mb;
  const int32_t avail = (int32_t)(avail64 > 128 ? 128 : avail64);
  const uint32_t lda2 = (uint32_t)(g.lda * 2);
  const int32_t skip = (int32_t)(m0 - mb);  // > 0 only when the whole wave is past M
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rr = 8 * i + (lane >> 3);
    int rel = rr + skip;
    if (rel > avail - 1) rel = avail - 1;
    const int u = (lane & 7) ^ swz(rr);
    aoff[i] = (uint32_t)rel * lda2 + 16u * (uint32_t)u;
  }
  return __builtin_amdgcn_make_buffer_rsrc((void *)abase, 0, 0x7fffffff, kBufferFlags);
}

__device__ __forceinline__ void zero_acc(floatx16 (&acc)[4][4]) {
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[mt][nt][v] = 0.0f;
}

// Epilogue: fp32 -> bf16 (RNE).  The MFMAs take the weight fragment as
// their first operand, so each accumulator tile is the transposed output
// block: lane l holds activation row m0 + 32mt + l%32 and output columns
// o0 + 32nt + 8j + 4g + i (i = 0..3) in registers 4j + i.  Four adjacent
// columns leave as one 8-byte store.  This is the path for outputs that do
// not take 16-byte stores (store_tile_lds takes the others).
__device__ __forceinline__ void store_tile(const GemmArgs &g, const floatx16 (&acc)[4][4],
                                           int64_t m0, int64_t o0, int jl, int grp) {
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

// Epilogue through LDS, for outputs that take 16-byte stores (16-byte
// aligned base, row stride a multiple of 8 elements).  Stores straight from
// the accumulator layout write 16-byte pieces of 32 rows per instruction;
// here each instruction writes 4 whole 256-byte rows of the wave's 128 x 128
// tile, 8 times fewer L2 write requests for the same bytes.
//  1. For each 32 x 32 accumulator tile, lanes l and l + 32 hold the two
//     8-byte halves of 16-byte chunks (8 columns) of row l % 32.  One
//     v_permlane32_swap per dword pairs them up: the lower lanes then hold
//     chunk j, the upper lanes chunk j + 1, whole.
//  2. The chunks go to the wave's own activation buffers (32 KB, idle after
//     the last step), row r at 256 B * r, chunk c at physical chunk
//     c ^ (r % 16): a 16-lane group of the ds_write_b128 covers 16 rows at
//     one chunk, one of the ds_read_b128 16 chunks of one row, both spread
//     over all banks.
//  3. Lane p reads row 4i + p / 16, chunk p % 16 and stores 16 bytes.  A
//     whole-width tile (o0 + 128 <= O) is read back whole first, then leaves
//     as 32 back-to-back buffer stores with no branch: the resource ends
//     after the wave's last row below M, so the hardware drops rows beyond
//     it.  Same-box A/B against reading and storing row by row with a test
//     per row: +1.1 % (70B gate) to +3.3 % (7B gate).  A tile with ragged
//     columns keeps the row-by-row stores.
__device__ __forceinline__ void store_tile_lds(const GemmArgs &g, const floatx16 (&acc)[4][4],
                                               u32x4 *lds, int64_t m0, int64_t o0, int lane) {
  // The lane's 32 + 32 LDS addresses below depend on nothing that changes
  // between tiles; an opaque copy of the lane index keeps the compiler from
  // hoisting them out of the tile loop, where they are spilled and reloaded
  // here, each reload waiting for every outstanding memory access.
  asm volatile("" : "+v"(lane));
  const int jl = lane & 31, grp = lane >> 5;
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int r = 32 * mt + jl;
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) {
      uint32_t lo[4], hi[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[j] = pack_bf16x2(acc[mt][nt][4 * j], acc[mt][nt][4 * j + 1]);
        hi[j] = pack_bf16x2(acc[mt][nt][4 * j + 2], acc[mt][nt][4 * j + 3]);
      }
#pragma unroll
      for (int jp = 0; jp < 4; jp += 2) {
        const auto a = __builtin_amdgcn_permlane32_swap(lo[jp], lo[jp + 1], false, false);
        const auto b = __builtin_amdgcn_permlane32_swap(hi[jp], hi[jp + 1], false, false);
        const uint32_t a0 = a[0], a1 = a[1], b0 = b[0], b1 = b[1];
        const int c = 4 * nt + jp + grp;
        lds[r * 16 + (c ^ (r & 15))] = (u32x4){a0, b0, a1, b1};
      }
    }
  }
  // The reads below take other lanes' writes: keep them after the writes.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLgkm0);
  asm volatile("" ::: "memory");
  const int c = lane & 15;
  if (o0 + kTileO <= g.O && g.ldo < ((int64_t)1 << 23)) {
    u32x4 v[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int r = 4 * i + (lane >> 4);
      v[i] = lds[r * 16 + (c ^ (r & 15))];
    }
    const int64_t left = g.M - m0;
    const int64_t rows = left <= 0 ? 0 : (left > 128 ? 128 : left);
    const uint32_t ldo2 = (uint32_t)(g.ldo * 2);  // < 2^24: every offset fits 32 bits
    const uint16_t *base = rows > 0 ? g.out + m0 * g.ldo + o0 : g.out;
    const int32_t nrec = rows > 0 ? (int32_t)((rows - 1) * ldo2 + kTileO * 2) : 0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, nrec, kBufferFlags);
    typedef unsigned int uvec4 __attribute__((ext_vector_type(4)));
    // Non-temporal: +0.4 to +0.8 % on 70B q and the 7B shapes, ±0.2 % on
    // the others, same box (the row-by-row stores had lost 23-45 % with it).
    constexpr int kStoreNt = 2;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t r = 4u * (uint32_t)i + (uint32_t)(lane >> 4);
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(uvec4, v[i]), rs,
                                             (int)(r * ldo2 + 16u * (uint32_t)c), 0, kStoreNt);
    }
    return;
  }
  const int64_t col = o0 + 8 * c;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const int r = 4 * i + (lane >> 4);
    const u32x4 v = lds[r * 16 + (c ^ (r & 15))];
    const int64_t m = m0 + r;
    if (m < g.M) {
      uint16_t *dst = g.out + m * g.ldo + col;
      if (col + 8 <= g.O) {
        *reinterpret_cast<u32x4 *>(dst) = v;
      } else {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (col + e < g.O) dst[e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

// The forward and input-gradient epilogue: through LDS when 16-byte stores
// fit.  For the input gradient, against its direct lane-paired stores
// (store_tile), same-box A/B, two rounds: 70B q +0.9-1.1 %, 70B down
// +1.5-3.5 %, 7B gate +1.5-4 %, summed gate/up +0.2-0.5 %.  (An earlier
// try measured -1 %: the compiler then hoisted the read-back addresses out
// of the tile loop and spilled 57 registers; store_tile_lds now keeps them
// in place.)
__device__ __forceinline__ void epilogue(const GemmArgs &g, const floatx16 (&acc)[4][4], int wave,
                                         int64_t m0, int64_t o0, int lane) {
  if (((reinterpret_cast<uintptr_t>(g.out) & 15) == 0) && ((g.ldo & 7) == 0))
    store_tile_lds(g, acc, &g_lds_a[wave][0][0], m0, o0, lane);
  else
    store_tile(g, acc, m0, o0, lane & 31, lane >> 5);
}

// Output tile `tile` of a forward launch: its rows, its group's output and
// weight, and its first output column.
__device__ __forceinline__ void fwd_tile(const GroupedArgs &ga, int tile, GemmArgs &g, int64_t &m0,
                                         int64_t &o0, int wave) {
  g = ga.base;
  int tm, to;
  map_tile(tile, g.tiles_m, ga.tiles_o, tm, to);
  // The group of output tile `to` (uniform; at most kMaxGroups iterations).
  int gi = 0;
  while (gi + 1 < ga.ngroups && to >= ga.grp[gi].tiles_o) {
    to -= ga.grp[gi].tiles_o;
    ++gi;
  }
  g.out = ga.grp[gi].out;
  g.ldo = ga.grp[gi].ldo;
  g.packed = ga.grp[gi].packed;
  g.am = ga.grp[gi].am;
  g.wn = ga.grp[gi].wn;
  g.O = ga.grp[gi].wn;
  m0 = (int64_t)tm * kTileM + wave * 128;
  o0 = (int64_t)to * kTileO;
}

// Forward: y_i = x . W_i^T.  The grid covers tiles_m x (output tiles of all
// groups); consecutive tiles share the activation rows (map_tile), also
// across a group boundary.  Work unit b < full_tiles is tile b; the units
// after it are the split-K slices of the remaining tiles (slice = unit %
// splits), each over split_steps reduction steps from step slice *
// split_steps, whose fp32 partials go to the workspace.
template <class Producer>
__global__ void __launch_bounds__(kGemmThreads, 1) nf4_gemm_fwd_kernel(const GroupedArgs ga) {
  const int T = ga.base.tiles_m * ga.tiles_o;
  const int U = ga.full_tiles + (T - ga.full_tiles) * ga.splits;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int jl = lane & 31;
  const int grp = lane >> 5;
#pragma unroll 1
  for (int b = blockIdx.x; b < U; b += gridDim.x) {
    int tile = b, slice = -1;
    if (b >= ga.full_tiles) {
      const int u = b - ga.full_tiles;
      tile = ga.full_tiles + u / ga.splits;
      slice = u - (u / ga.splits) * ga.splits;
    }
    GemmArgs g;
    int64_t m0, o0;
    fwd_tile(ga, tile, g, m0, o0, wave);
    if (slice >= 0) {
      const int64_t steps = g.R / kStep;
      g.k0 = (int64_t)slice * ga.split_steps;
      const int64_t left = steps - g.k0;
      g.R = kStep * (left < ga.split_steps ? left : ga.split_steps);
    }
    uint32_t aoff[16];
    const __amdgpu_buffer_rsrc_t arsrc = activation_setup(g, m0, lane, aoff);
    Producer prod;
    prod.init(g, o0, (uint32_t)(uintptr_t)(lds_void_t *)&g_lds_b[0][0]);
    floatx16 acc[4][4];
    zero_acc(acc);
    gemm_main<Producer>(g, prod, acc, &g_lds_a[wave][0][0], &g_lds_a[wave][1][0], g_lds_b[0],
                        g_lds_b[1], arsrc, aoff, (int)(g.R / kStep), jl, grp);
    if (slice < 0) {
      epilogue(g, acc, wave, m0, o0, lane);
    } else {
      floatx4 *part = reinterpret_cast<floatx4 *>(
          ga.ws + (int64_t)(b - ga.full_tiles) * kPartialFloats) + threadIdx.x;
#pragma unroll
      for (int i = 0; i < 64; ++i) {
        const floatx16 &a = acc[i >> 4][(i >> 2) & 3];
        const int v = 4 * (i & 3);
        part[i * kGemmThreads] = (floatx4){a[v], a[v + 1], a[v + 2], a[v + 3]};
      }
    }
  }
}

// Split-K fixup, launched after the main kernel on the same stream.  The
// partials of a unit are [quad i = 0..63][thread t] floatx4, quad i holding
// thread t's acc[i / 16][(i / 4) % 4][4 (i % 4) .. + 3]: 4 adjacent output
// columns of one row.  Workgroup (j, q) sums quads kFixupQuads * q .. of tail
// tile full_tiles + j over its `splits` slices in slice order (fp32) and
// stores them as bf16, so that 16 workgroups per tile keep every CU loading.
constexpr int kFixupQuads = 4;
constexpr int kFixupBlocksPerTile = 64 / kFixupQuads;
template <bool kDgrad>
__global__ void __launch_bounds__(kGemmThreads) nf4_gemm_fixup_kernel(const GroupedArgs ga) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x / kFixupBlocksPerTile;
  const int q = blockIdx.x - j * kFixupBlocksPerTile;
  GemmArgs g;
  int64_t m0, o0;
  if constexpr (kDgrad) {
    // The input gradient's tile: rows and columns of dx (ga.base.out).
    g = ga.base;
    int tm, to;
    map_tile(ga.full_tiles + j, g.tiles_m, g.tiles_o, tm, to);
    m0 = (int64_t)tm * kTileM + wave * 128;
    o0 = (int64_t)to * kTileO;
  } else {
    fwd_tile(ga, ga.full_tiles + j, g, m0, o0, wave);
  }
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(g.out) & 7) == 0) && ((g.ldo & 3) == 0);
  const floatx4 *part = reinterpret_cast<const floatx4 *>(ga.ws + (int64_t)j * ga.splits *
                                                                      kPartialFloats) +
                        threadIdx.x;
  // All quads of a slice are loaded before any is added, so each thread has
  // kFixupQuads (x2 with the unroll) loads in flight rather than one.
  floatx4 acc[kFixupQuads];
#pragma unroll
  for (int ii = 0; ii < kFixupQuads; ++ii) acc[ii] = (floatx4){0.f, 0.f, 0.f, 0.f};
#pragma unroll 2
  for (int sl = 0; sl < ga.splits; ++sl) {
    floatx4 p[kFixupQuads];
#pragma unroll
    for (int ii = 0; ii < kFixupQuads; ++ii)
      p[ii] = part[(int64_t)sl * (kPartialFloats / 4) + (q * kFixupQuads + ii) * kGemmThreads];
#pragma unroll
    for (int ii = 0; ii < kFixupQuads; ++ii) {
      acc[ii][0] += p[ii][0];
      acc[ii][1] += p[ii][1];
      acc[ii][2] += p[ii][2];
      acc[ii][3] += p[ii][3];
    }
  }
  // Whole-width tile with 16-byte stores: lanes l and l + 32 pair their
  // halves (as store_tile does) and store 16-byte chunks through a buffer
  // resource that ends after the wave's last row below M.  70B k alone:
  // +1.4 % for the whole split launch.
  if (((reinterpret_cast<uintptr_t>(g.out) & 15) == 0) && ((g.ldo & 7) == 0) &&
      o0 + kTileO <= g.O && g.ldo < ((int64_t)1 << 23)) {
    const int64_t left = g.M - m0;
    const int64_t rows = left <= 0 ? 0 : (left > 128 ? 128 : left);
    const uint32_t ldo2 = (uint32_t)(g.ldo * 2);
    const uint16_t *base = rows > 0 ? g.out + m0 * g.ldo + o0 : g.out;
    const int32_t nrec = rows > 0 ? (int32_t)((rows - 1) * ldo2 + kTileO * 2) : 0;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)base, 0, nrec, kBufferFlags);
    typedef unsigned int uvec4 __attribute__((ext_vector_type(4)));
    const int i0 = q * kFixupQuads;  // quads i0..i0+3: one (mt, nt), j = 0..3
    const uint32_t rowoff = (uint32_t)(32 * (i0 >> 4) + (lane & 31)) * ldo2;
#pragma unroll
    for (int jp = 0; jp < 4; jp += 2) {
      const uint32_t lo0 = pack_bf16x2(acc[jp][0], acc[jp][1]);
      const uint32_t hi0 = pack_bf16x2(acc[jp][2], acc[jp][3]);
      const uint32_t lo1 = pack_bf16x2(acc[jp + 1][0], acc[jp + 1][1]);
      const uint32_t hi1 = pack_bf16x2(acc[jp + 1][2], acc[jp + 1][3]);
      const auto a = __builtin_amdgcn_permlane32_swap(lo0, lo1, false, false);
      const auto b = __builtin_amdgcn_permlane32_swap(hi0, hi1, false, false);
      const uint32_t a0 = a[0], a1 = a[1], b0 = b[0], b1 = b[1];
      const int c = 4 * ((i0 >> 2) & 3) + jp + (lane >> 5);
      __builtin_amdgcn_raw_buffer_store_b128((uvec4){a0, b0, a1, b1}, rs,
                                             (int)(rowoff + 16u * (uint32_t)c), 0, 0);
    }
    return;
  }
#pragma unroll
  for (int ii = 0; ii < kFixupQuads; ++ii) {
    const int i = q * kFixupQuads + ii;
    const int64_t m = m0 + 32 * (i >> 4) + (lane & 31);
    const int64_t c = o0 + 4 * (lane >> 5) + 32 * ((i >> 2) & 3) + 8 * (i & 3);
    if (m >= g.M || c >= g.O) continue;
    uint16_t *o = g.out + m * g.ldo + c;
    const uint32_t lo = pack_bf16x2(acc[ii][0], acc[ii][1]);
    const uint32_t hi = pack_bf16x2(acc[ii][2], acc[ii][3]);
    if (vec_ok && c + 4 <= g.O) {
      *reinterpret_cast<u32x2 *>(o) = (u32x2){lo, hi};
    } else {
      o[0] = (uint16_t)(lo & 0xffffu);
      if (c + 1 < g.O) o[1] = (uint16_t)(lo >> 16);
      if (c + 2 < g.O) o[2] = (uint16_t)(hi & 0xffffu);
      if (c + 3 < g.O) o[3] = (uint16_t)(hi >> 16);
    }
  }
}

// silu(x) = x / (1 + e^-x) (doublepass/src/math.rs:91-93) in fp32, with the
// hardware base-2 exponential and reciprocal: x * rcp(1 + 2^(-x log2 e)).
__device__ __forceinline__ float silu(float x) {
  const float e = __builtin_amdgcn_exp2f(-x * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}

// SwiGLU epilogue: accumulator tiles nt = 0, 1 hold gate columns c0 + 32nt +
// 8j + 4g + i, tiles nt + 2 the up columns with the same index (the weight
// tile's rows 64-127 are the up rows), so hidden = silu(gate) * up is
// elementwise within a lane.  Four adjacent hidden columns leave as one
// 8-byte store.
__device__ __forceinline__ void store_swiglu(const GemmArgs &g, const floatx16 (&acc)[4][4],
                                             int64_t m0, int64_t c0, int jl, int grp) {
  const bool vec_ok = ((reinterpret_cast<uintptr_t>(g.out) & 7) == 0) && ((g.ldo & 3) == 0);
  const int64_t cl = g.O - (c0 + 4 * grp);
  const int32_t clim = (int32_t)(cl < 0 ? 0 : (cl > (1 << 30) ? (1 << 30) : cl));
#pragma unroll
  for (int mt = 0; mt < 4; ++mt) {
    const int64_t m = m0 + 32 * mt + jl;
    if (m < g.M) {
      uint16_t *orow = g.out + m * g.ldo + c0 + 4 * grp;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int c = 32 * nt + 8 * j;
          float h[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            h[i] = silu(acc[mt][nt][4 * j + i]) * acc[mt][nt + 2][4 * j + i];
          const uint32_t lo = pack_bf16x2(h[0], h[1]);
          const uint32_t hi = pack_bf16x2(h[2], h[3]);
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

// Forward with the SwiGLU of single_layer_forward fused into the epilogue
// (doublepass/src/forward.rs:251-254): hidden = silu(x . Wg^T) * (x . Wu^T).
// A tile is 512 rows x 64 hidden columns c0..c0+63; its weight tile holds
// gate rows c0..c0+63 (produced by waves 0-1) and up rows c0..c0+63 (waves
// 2-3), so each tile does the MFMA work of a 128-column tile and writes half
// the output bytes.  grp[0] is the gate weight, grp[1] the up weight.
template <class Producer>
__global__ void __launch_bounds__(kGemmThreads, 1) nf4_gemm_swiglu_kernel(const GroupedArgs ga) {
  const int T = ga.base.tiles_m * ga.tiles_o;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int jl = lane & 31;
  const int grp = lane >> 5;
  const GemmGroup &gw = ga.grp[wave < 2 ? 0 : 1];
#pragma unroll 1
  for (int b = blockIdx.x; b < T; b += gridDim.x) {
    const GemmArgs &g = ga.base;
    int tm, th;
    map_tile(b, g.tiles_m, ga.tiles_o, tm, th);
    const int64_t m0 = (int64_t)tm * kTileM + wave * 128;
    const int64_t c0 = (int64_t)th * (kTileO / 2);
    uint32_t aoff[16];
    const __amdgpu_buffer_rsrc_t arsrc = activation_setup(g, m0, lane, aoff);
    // This wave's weight: tile rows 0-63 are gate rows c0 + r, rows 64-127
    // up rows c0 + r - 64.
    GemmArgs gp = g;
    gp.packed = gw.packed;
    gp.am = gw.am;
    gp.wn = gw.wn;
    Producer prod;
    prod.init(gp, wave < 2 ? c0 : c0 - 64, (uint32_t)(uintptr_t)(lds_void_t *)&g_lds_b[0][0]);
    floatx16 acc[4][4];
    zero_acc(acc);
    gemm_main<Producer>(g, prod, acc, &g_lds_a[wave][0][0], &g_lds_a[wave][1][0], g_lds_b[0],
                        g_lds_b[1], arsrc, aoff, (int)(g.R / kStep), jl, grp);
    store_swiglu(g, acc, m0, c0, jl, grp);
  }
}

// Input gradient: dx = sum_i dy_i . W_i, the groups run one after another
// into the same accumulator.  Between two groups no barrier is needed: every
// read of the shared weight tiles ended before the last step's barrier, and
// the activation buffers are per wave.  The reduction of a tile is the
// groups' steps in order (group i's W rows 64 s .. 64 s + 63 at step s).
// Work unit b < full_tiles is tile b; the units after it are split-K slices
// of the remaining tiles (slice = unit % splits), each over split_steps of
// that step sequence (its part of each group it meets), whose fp32 partials
// go to the workspace and are summed by nf4_gemm_fixup_kernel<true>.  The
// launch without a split runs the kSplit = false instantiation, which keeps
// none of the slice bookkeeping (the split one spills a few registers per
// tile).
template <class Producer, bool kSplit>
__global__ void __launch_bounds__(kGemmThreads, 1) nf4_gemm_dgrad_kernel(const GroupedArgs ga) {
  const int T = ga.base.tiles_m * ga.base.tiles_o;
  const int U = kSplit ? ga.full_tiles + (T - ga.full_tiles) * ga.splits : T;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const int jl = lane & 31;
  const int grp = lane >> 5;
  // Reduction steps over all groups (check_offsets bounds each group's below
  // 2^16).
  int total = 0;
  if constexpr (kSplit)
    for (int gi = 0; gi < ga.ngroups; ++gi) total += (int)(ga.grp[gi].wn / kStep);
#pragma unroll 1
  for (int b = blockIdx.x; b < U; b += gridDim.x) {
    int tile = b, slice = -1;
    if (kSplit && b >= ga.full_tiles) {
      const int u = b - ga.full_tiles;
      tile = ga.full_tiles + u / ga.splits;
      slice = u - (u / ga.splits) * ga.splits;
    }
    GemmArgs g = ga.base;
    int tm, to;
    map_tile(tile, g.tiles_m, g.tiles_o, tm, to);
    const int64_t m0 = (int64_t)tm * kTileM + wave * 128;
    const int64_t o0 = (int64_t)to * kTileO;
    floatx16 acc[4][4];
    zero_acc(acc);
    if constexpr (!kSplit) {
#pragma unroll 1
      for (int gi = 0; gi < ga.ngroups; ++gi) {
        g.a = ga.grp[gi].a;
        g.lda = ga.grp[gi].lda;
        g.packed = ga.grp[gi].packed;
        g.am = ga.grp[gi].am;
        g.wn = ga.grp[gi].wn;
        g.R = ga.grp[gi].wn;
        uint32_t aoff[16];
        const __amdgpu_buffer_rsrc_t arsrc = activation_setup(g, m0, lane, aoff);
        Producer prod;
        prod.init(g, o0, (uint32_t)(uintptr_t)(lds_void_t *)&g_lds_b[0][0]);
        gemm_main<Producer>(g, prod, acc, &g_lds_a[wave][0][0], &g_lds_a[wave][1][0],
                            g_lds_b[0], g_lds_b[1], arsrc, aoff, (int)(g.R / kStep), jl, grp);
      }
      epilogue(g, acc, wave, m0, o0, lane);
    } else {
      int s_lo = 0, s_hi = total;
      if (slice >= 0) {
        s_lo = slice * ga.split_steps;
        s_hi = (s_lo + ga.split_steps < total) ? s_lo + ga.split_steps : total;
      }
      int gbase = 0;  // first step of group gi
#pragma unroll 1
      for (int gi = 0; gi < ga.ngroups; ++gi) {
        const int steps = (int)(ga.grp[gi].wn / kStep);
        const int lo = (s_lo > gbase) ? s_lo : gbase;
        const int hi = (s_hi < gbase + steps) ? s_hi : gbase + steps;
        if (lo < hi) {
          g.a = ga.grp[gi].a;
          g.lda = ga.grp[gi].lda;
          g.packed = ga.grp[gi].packed;
          g.am = ga.grp[gi].am;
          g.wn = ga.grp[gi].wn;
          g.k0 = lo - gbase;
          g.R = (int64_t)kStep * (hi - lo);
          uint32_t aoff[16];
          const __amdgpu_buffer_rsrc_t arsrc = activation_setup(g, m0, lane, aoff);
          Producer prod;
          prod.init(g, o0, (uint32_t)(uintptr_t)(lds_void_t *)&g_lds_b[0][0]);
          gemm_main<Producer>(g, prod, acc, &g_lds_a[wave][0][0], &g_lds_a[wave][1][0],
                              g_lds_b[0], g_lds_b[1], arsrc, aoff, hi - lo, jl, grp);
        }
        gbase += steps;
      }
      if (slice < 0) {
        epilogue(g, acc, wave, m0, o0, lane);
      } else {
        floatx4 *part = reinterpret_cast<floatx4 *>(
            ga.ws + (int64_t)(b - ga.full_tiles) * kPartialFloats) + threadIdx.x;
#pragma unroll
        for (int i = 0; i < 64; ++i) {
          const floatx16 &a = acc[i >> 4][(i >> 2) & 3];
          const int v = 4 * (i & 3);
          part[i * kGemmThreads] = (floatx4){a[v], a[v + 1], a[v + 2], a[v + 3]};
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
  a.block_shift = t.block_size > 64 ? group_shift(t.block_size / 64) : 0;
  return a;
}

// Shared argument checks of the two GEMM entry points.  W is [wn, wk].  With
// m == 0 (no tokens) nothing is read or written: the activation and output
// pointers may be NULL or unaligned (an empty tensor's or vector's data
// pointer), and only the weight's shape is checked.
static int32_t check_gemm(const uint16_t *act, const nf4s_tensor *w, int64_t m, int64_t wn,
                          int64_t wk, const uint16_t *out) {
  if (m != 0 && (act == nullptr || out == nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "activation or output is NULL");
  if (m < 0 || wn <= 0 || wk <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad GEMM shape m=%lld n=%lld k=%lld",
                (long long)m, (long long)wn, (long long)wk);
  // Tile counts are 32-bit: (dim + 511) / 512 must fit before the launch
  // code bounds the tile total.
  constexpr int64_t kMaxDim = (int64_t)1 << 39;
  if (m > kMaxDim || wn > kMaxDim || wk > kMaxDim)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "GEMM dimension beyond 2^39: m=%lld n=%lld k=%lld",
                (long long)m, (long long)wn, (long long)wk);
  int64_t numel;
  if (__builtin_mul_overflow(wn, wk, &numel))
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "weight of %lld x %lld elements overflows 64 bits",
                (long long)wn, (long long)wk);
  const int32_t rc = validate_tensor(w, numel);
  if (rc != NF4S_OK) return rc;
  // A 64-deep reduction step must lie in one absmax block: block sizes 64,
  // 128, 256, ... (64 << s), with whole blocks per row.
  const int32_t bsz = w->block_size;
  if (bsz < 64 || bsz > (1 << 20) || (bsz & (bsz - 1)) != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                "fused GEMM needs block_size 64 << s (64, 128, 256, ...), got %d", bsz);
  if (wk % 64 != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "fused GEMM needs k %% 64 == 0, got %lld",
                (long long)wk);
  if (wk % bsz != 0)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                "fused GEMM needs k %% block_size == 0 (whole blocks per row), got k %lld, "
                "block_size %d", (long long)wk, bsz);
  if (m == 0) return NF4S_OK;
  if (!aligned(act, 16) || !aligned(w->packed, 16))
    return fail(NF4S_ERR_MISALIGNED, "activation and packed weights must be 16-byte aligned");
  if (!aligned(out, 2)) return fail(NF4S_ERR_MISALIGNED, "output must be 2-byte aligned");
  return NF4S_OK;
}

// The activation loads address a wave's 128 rows with 32-bit offsets.  The
// bound also keeps the kernels' 32-bit step counts (R / 64 <= 2^16) exact.
static int32_t check_offsets(int64_t lda) {
  if (lda > (int64_t)1 << 22)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "activation row of %lld elements is too long",
                (long long)lda);
  return NF4S_OK;
}

// A forward group can take the batched weight loads: whole 4-block absmax
// groups per row (k % 256), aligned group loads, and 4-block groups inside
// one double-quant scale.
static bool fwd_batchable(const nf4s_tensor &w, int64_t k) {
  if (k % 256 != 0 || w.block_size != 64) return false;
  if (w.absmax_q != nullptr) return aligned(w.absmax_q, 4) && w.dq_group >= 4;
  return aligned(w.absmax, 16);
}

static GemmGroup group_of(const nf4s_tensor &w, int64_t wn) {
  GemmGroup q{};
  q.packed = w.packed;
  q.am = absmax_of(w);
  q.wn = wn;
  return q;
}

// Split-K plan for a forward launch of T tiles and `nsteps` reduction steps.
// A last round of r tiles (0 < r <= half the CUs) runs as S = CUs / r
// slices per tile, so that it fills the chip; every slice keeps at least
// `unroll` steps (and a multiple of them).  Returns the partial-tile count
// r * S, or 0 for no split.
struct SplitPlan {
  int64_t tail_tiles, splits, split_steps;
};
static SplitPlan split_plan(int64_t T, int64_t nsteps, int unroll) {
  SplitPlan p{0, 1, 0};
  const int64_t cus = cu_slots();
  const int64_t r = T % cus;
  if (r == 0 || 2 * r > cus) return p;
  int64_t S = cus / r;
  if (S > nsteps / unroll) S = nsteps / unroll;
  if (S < 2) return p;
  int64_t per = (nsteps + S - 1) / S;
  per = (per + unroll - 1) / unroll * unroll;
  S = (nsteps + per - 1) / per;
  if (S < 2) return p;
  p.tail_tiles = r;
  p.splits = S;
  p.split_steps = per;
  return p;
}

// Workspace bytes a split plan needs (0 without a split).
static int64_t split_bytes(const SplitPlan &p) {
  return p.tail_tiles * p.splits * kPartialFloats * (int64_t)sizeof(float);
}

template <class Producer>
static int32_t launch_fwd(GroupedArgs &ga, hipStream_t s, void *ws, int64_t ws_bytes) {
  const int64_t T = (int64_t)ga.base.tiles_m * ga.tiles_o;
  if (T == 0) return NF4S_OK;
  if (T > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
  ga.full_tiles = (int32_t)T;
  ga.splits = 1;
  ga.split_steps = 0;
  ga.ws = nullptr;
  const SplitPlan p = split_plan(T, ga.base.R / kStep, Producer::kUnroll);
  if (ws != nullptr && p.tail_tiles > 0 && ws_bytes >= split_bytes(p)) {
    ga.full_tiles = (int32_t)(T - p.tail_tiles);
    ga.splits = (int32_t)p.splits;
    ga.split_steps = (int32_t)p.split_steps;
    ga.ws = static_cast<float *>(ws);
  }
  const int64_t U = ga.full_tiles + (T - ga.full_tiles) * ga.splits;
  hipLaunchKernelGGL(nf4_gemm_fwd_kernel<Producer>, dim3(persistent_grid(U)), dim3(kGemmThreads),
                     0, s, ga);
  int32_t rc = check_launch("nf4_gemm_fwd");
  if (rc == NF4S_OK && ga.splits > 1) {
    hipLaunchKernelGGL(nf4_gemm_fixup_kernel<false>,
                       dim3((uint32_t)((T - ga.full_tiles) * kFixupBlocksPerTile)),
                       dim3(kGemmThreads), 0, s, ga);
    rc = check_launch("nf4_gemm_fixup");
  }
  return rc;
}

// Reduction steps of an input-gradient launch: its groups' steps in order.
static int64_t dgrad_steps(const int64_t *ns, int32_t count) {
  int64_t steps = 0;
  for (int32_t i = 0; i < count; ++i) steps += ns[i] / kStep;
  return steps;
}

template <class Producer>
static int32_t launch_dgrad(GroupedArgs &ga, int64_t nsteps, hipStream_t s, void *ws,
                            int64_t ws_bytes) {
  const int64_t T = (int64_t)ga.base.tiles_m * ga.base.tiles_o;
  if (T == 0) return NF4S_OK;
  if (T > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
  ga.full_tiles = (int32_t)T;
  ga.splits = 1;
  ga.split_steps = 0;
  ga.ws = nullptr;
  const SplitPlan p = split_plan(T, nsteps, Producer::kUnroll);
  if (ws != nullptr && p.tail_tiles > 0 && ws_bytes >= split_bytes(p)) {
    ga.full_tiles = (int32_t)(T - p.tail_tiles);
    ga.splits = (int32_t)p.splits;
    ga.split_steps = (int32_t)p.split_steps;
    ga.ws = static_cast<float *>(ws);
  }
  const int64_t U = ga.full_tiles + (T - ga.full_tiles) * ga.splits;
  if (ga.splits > 1)
    hipLaunchKernelGGL((nf4_gemm_dgrad_kernel<Producer, true>), dim3(persistent_grid(U)),
                       dim3(kGemmThreads), 0, s, ga);
  else
    hipLaunchKernelGGL((nf4_gemm_dgrad_kernel<Producer, false>), dim3(persistent_grid(U)),
                       dim3(kGemmThreads), 0, s, ga);
  int32_t rc = check_launch("nf4_gemm_dgrad");
  if (rc == NF4S_OK && ga.splits > 1) {
    hipLaunchKernelGGL(nf4_gemm_fixup_kernel<true>,
                       dim3((uint32_t)((T - ga.full_tiles) * kFixupBlocksPerTile)),
                       dim3(kGemmThreads), 0, s, ga);
    rc = check_launch("nf4_gemm_fixup");
  }
  return rc;
}

// Workspace bytes the split-K input gradient over these weights needs (0: no
// split), for either producer's step granularity.
static int64_t dgrad_workspace_bytes(const int64_t *ns, int32_t count, int64_t m, int64_t k) {
  constexpr int64_t kMaxDim = (int64_t)1 << 39;  // beyond it the GEMM rejects the shape
  if (m <= 0 || m > kMaxDim || k <= 0 || k > kMaxDim || k % 64 != 0) return 0;
  for (int32_t i = 0; i < count; ++i)
    if (ns[i] <= 0 || ns[i] > kMaxDim || ns[i] % 64 != 0) return 0;
  const int64_t T = ((m + kTileM - 1) / kTileM) * ((k + kTileO - 1) / kTileO);
  const int64_t steps = dgrad_steps(ns, count);
  int64_t best = 0;
  for (int unroll : {2, 4}) {
    const int64_t b = split_bytes(split_plan(T, steps, unroll));
    if (b > best) best = b;
  }
  return best;
}


// Forward over `count` weights W_i [ns[i], k] sharing x [m, k]: y_i = x . W_i^T.
// Weights of one kind (double-quantized or not, batched loads or not) share
// a launch; a mixed set runs as one launch per kind.
static int32_t gemm_fwd_groups(const uint16_t *x, const nf4s_tensor *ws, const int64_t *ns,
                               uint16_t *const *ys, int32_t count, int64_t m, int64_t k,
                               hipStream_t s, void *work = nullptr, int64_t work_bytes = 0) {
  if (count <= 0 || count > kMaxGroups)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "count must be 1..%d, got %d", kMaxGroups, count);
  if (ws == nullptr || ns == nullptr || ys == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "weights, sizes or outputs are NULL");
  int32_t rc = NF4S_OK;
  for (int32_t i = 0; i < count && rc == NF4S_OK; ++i)
    rc = check_gemm(x, &ws[i], m, ns[i], k, ys[i]);
  if (rc == NF4S_OK) rc = check_offsets(k);
  if (rc != NF4S_OK) return rc;
  if (m == 0) return NF4S_OK;
  // Kind of each weight: bit 0 double-quant, bit 1 batched loads.
  int kind[kMaxGroups];
  for (int32_t i = 0; i < count; ++i)
    kind[i] = (ws[i].absmax_q != nullptr ? 1 : 0) | (fwd_batchable(ws[i], k) ? 2 : 0);
  bool done[kMaxGroups] = {false, false, false, false};
  for (int32_t i = 0; i < count; ++i) {
    if (done[i]) continue;
    GroupedArgs ga{};
    GemmArgs &g = ga.base;
    g.a = x;
    g.lda = k;
    g.M = m;
    g.R = k;
    g.wk = k;
    g.tiles_m = (int32_t)((m + kTileM - 1) / kTileM);
    int64_t tiles = 0;
    for (int32_t j = i; j < count; ++j) {
      if (done[j] || kind[j] != kind[i]) continue;
      GemmGroup q = group_of(ws[j], ns[j]);
      q.out = ys[j];
      q.ldo = ns[j];
      q.tiles_o = (int32_t)((ns[j] + kTileO - 1) / kTileO);
      tiles += q.tiles_o;
      ga.grp[ga.ngroups++] = q;
      done[j] = true;
    }
    if (tiles > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
    ga.tiles_o = (int32_t)tiles;
    switch (kind[i]) {
      case 3: rc = launch_fwd<FwdBatchProducer<true>>(ga, s, work, work_bytes); break;
      case 2: rc = launch_fwd<FwdBatchProducer<false>>(ga, s, work, work_bytes); break;
      case 1: rc = launch_fwd<FwdProducer<true>>(ga, s, work, work_bytes); break;
      default: rc = launch_fwd<FwdProducer<false>>(ga, s, work, work_bytes); break;
    }
    if (rc != NF4S_OK) return rc;
  }
  return NF4S_OK;
}

// hidden [m, ff] = silu(x . Wg^T) * (x . Wu^T), Wg and Wu [ff, k] of one kind.
static int32_t gemm_swiglu(const uint16_t *x, const nf4s_tensor *wg, const nf4s_tensor *wu,
                           int64_t m, int64_t ff, int64_t k, uint16_t *hidden, hipStream_t s) {
  if (wg == nullptr || wu == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "weight descriptor is NULL");
  int32_t rc = check_gemm(x, wg, m, ff, k, hidden);
  if (rc == NF4S_OK) rc = check_gemm(x, wu, m, ff, k, hidden);
  if (rc == NF4S_OK) rc = check_offsets(k);
  if (rc != NF4S_OK) return rc;
  const bool dq = wg->absmax_q != nullptr;
  const bool batch = fwd_batchable(*wg, k) && fwd_batchable(*wu, k);
  if ((wu->absmax_q != nullptr) != dq)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                "gate and up weights must both be double-quantized or both not");
  if (m == 0) return NF4S_OK;
  GroupedArgs ga{};
  GemmArgs &g = ga.base;
  g.a = x;
  g.lda = k;
  g.out = hidden;
  g.ldo = ff;
  g.M = m;
  g.O = ff;
  g.R = k;
  g.wk = k;
  g.tiles_m = (int32_t)((m + kTileM - 1) / kTileM);
  const int64_t tiles_h = (ff + kTileO / 2 - 1) / (kTileO / 2);
  if ((int64_t)g.tiles_m * tiles_h > 0x7fffffff)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
  ga.tiles_o = (int32_t)tiles_h;
  ga.grp[0] = group_of(*wg, ff);
  ga.grp[1] = group_of(*wu, ff);
  ga.ngroups = 2;
  const uint32_t grid = persistent_grid((int64_t)g.tiles_m * tiles_h);
  if (batch && dq)
    hipLaunchKernelGGL(nf4_gemm_swiglu_kernel<FwdBatchProducer<true>>, dim3(grid),
                       dim3(kGemmThreads), 0, s, ga);
  else if (batch)
    hipLaunchKernelGGL(nf4_gemm_swiglu_kernel<FwdBatchProducer<false>>, dim3(grid),
                       dim3(kGemmThreads), 0, s, ga);
  else if (dq)
    hipLaunchKernelGGL(nf4_gemm_swiglu_kernel<FwdProducer<true>>, dim3(grid), dim3(kGemmThreads),
                       0, s, ga);
  else
    hipLaunchKernelGGL(nf4_gemm_swiglu_kernel<FwdProducer<false>>, dim3(grid),
                       dim3(kGemmThreads), 0, s, ga);
  return check_launch("nf4_gemm_swiglu");
}

// Input gradient dx [m, k] = sum_i dy_i [m, ns[i]] . W_i [ns[i], k].
static int32_t gemm_dgrad_groups(const uint16_t *const *dys, const nf4s_tensor *ws,
                                 const int64_t *ns, int32_t count, int64_t m, int64_t k,
                                 uint16_t *dx, hipStream_t s, void *work = nullptr,
                                 int64_t work_bytes = 0) {
  if (count <= 0 || count > kMaxGroups)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "count must be 1..%d, got %d", kMaxGroups, count);
  if (dys == nullptr || ws == nullptr || ns == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "gradients, weights or sizes are NULL");
  const bool dq = ws[0].absmax_q != nullptr;
  for (int32_t i = 0; i < count; ++i) {
    int32_t rc = check_gemm(dys[i], &ws[i], m, ns[i], k, dx);
    if (rc == NF4S_OK) rc = check_offsets(ns[i]);
    if (rc != NF4S_OK) return rc;
    if (ns[i] % 64 != 0)
      return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "dgrad needs n %% 64 == 0, got %lld",
                  (long long)ns[i]);
    if ((ws[i].absmax_q != nullptr) != dq)
      return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                  "summed dgrad needs all weights double-quantized or none");
  }
  if (m == 0) return NF4S_OK;
  GroupedArgs ga{};
  GemmArgs &g = ga.base;
  g.out = dx;
  g.ldo = k;
  g.M = m;
  g.O = k;
  g.wk = k;
  g.tiles_m = (int32_t)((m + kTileM - 1) / kTileM);
  g.tiles_o = (int32_t)((k + kTileO - 1) / kTileO);
  for (int32_t i = 0; i < count; ++i) {
    GemmGroup q = group_of(ws[i], ns[i]);
    q.a = dys[i];
    q.lda = ns[i];
    ga.grp[ga.ngroups++] = q;
  }
  // Batched absmax loads: whole 4-step groups for every weight, both blocks
  // of a 128-column tile in every row (k % 128), aligned pair loads, and
  // the two blocks of a pair inside one double-quant scale group.
  bool batch = k % 128 == 0;
  for (int32_t i = 0; i < count && batch; ++i) {
    batch = ns[i] % 256 == 0 && ws[i].block_size == 64;
    if (dq)
      batch = batch && aligned(ws[i].absmax_q, 2) && ws[i].dq_group >= 2;
    else
      batch = batch && aligned(ws[i].absmax, 8);
  }
  const int64_t nsteps = dgrad_steps(ns, count);
  if (batch)
    return dq ? launch_dgrad<DgradBatchProducer<true>>(ga, nsteps, s, work, work_bytes)
              : launch_dgrad<DgradBatchProducer<false>>(ga, nsteps, s, work, work_bytes);
  return dq ? launch_dgrad<DgradProducer<true>>(ga, nsteps, s, work, work_bytes)
            : launch_dgrad<DgradProducer<false>>(ga, nsteps, s, work, work_bytes);
}

// Workspace bytes the split-K forward over these weights needs (0: no split
// would help, or a shape the GEMM itself rejects, which the GEMM reports).
// Weights of one kind share a launch and a mixed set runs one launch per
// kind, so this is the largest plan over every subset of the weights and
// both producers' step multiples: enough for any partition into launches.
static int64_t fwd_workspace_bytes(const int64_t *ns, int32_t count, int64_t m, int64_t k) {
  constexpr int64_t kMaxDim = (int64_t)1 << 39;  // beyond it the GEMM rejects the shape
  if (m <= 0 || m > kMaxDim || k <= 0 || k > kMaxDim || k % 64 != 0) return 0;
  for (int32_t i = 0; i < count; ++i)
    if (ns[i] <= 0 || ns[i] > kMaxDim) return 0;
  const int64_t tiles_m = (m + kTileM - 1) / kTileM;
  int64_t best = 0;
  for (uint32_t set = 1; set < (1u << count); ++set) {
    int64_t tiles_o = 0;
    for (int32_t i = 0; i < count; ++i)
      if (set & (1u << i)) tiles_o += (ns[i] + kTileO - 1) / kTileO;
    const int64_t T = tiles_m * tiles_o;
    for (int unroll : {2, 4}) {
      const int64_t b = split_bytes(split_plan(T, k / kStep, unroll));
      if (b > best) best = b;
    }
  }
  return best;
}

static_assert(kPartialFloats * (int64_t)sizeof(float) == kGemmPartialTileBytes,
              "partial tile size shared with nf4_noalloc.hip");

int32_t fwd_workspace_query(const int64_t *ns, int32_t count, int64_t m, int64_t k,
                            int64_t *bytes) {
  if (bytes == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bytes is NULL");
  *bytes = 0;
  if (count <= 0 || count > kMaxGroups || ns == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "count must be 1..%d with sizes", kMaxGroups);
  *bytes = fwd_workspace_bytes(ns, count, m, k);
  return NF4S_OK;
}

int32_t gemm_fwd_grouped_on(const uint16_t *x, const nf4s_tensor *ws, const int64_t *ns,
                            uint16_t *const *ys, int32_t count, int64_t m, int64_t k,
                            hipStream_t s, void *work, int64_t work_bytes) {
  return gemm_fwd_groups(x, ws, ns, ys, count, m, k, s, work, work_bytes);
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

int32_t nf4s_gemm_fwd(const uint16_t *x, const nf4s_tensor *w, int64_t m, int64_t n, int64_t k,
                      uint16_t *y, void *stream) {
  clear_error();
  if (w == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "weight descriptor is NULL");
  uint16_t *ys[1] = {y};
  return gemm_fwd_groups(x, w, &n, ys, 1, m, k, as_stream(stream));
}

int32_t nf4s_gemm_dgrad(const uint16_t *dy, const nf4s_tensor *w, int64_t m, int64_t n,
                        int64_t k, uint16_t *dx, void *stream) {
  clear_error();
  if (w == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "weight descriptor is NULL");
  const uint16_t *dys[1] = {dy};
  return gemm_dgrad_groups(dys, w, &n, 1, m, k, dx, as_stream(stream));
}

int32_t nf4s_gemm_fwd_grouped(const uint16_t *x, const nf4s_tensor *ws, const int64_t *ns,
                              uint16_t *const *ys, int32_t count, int64_t m, int64_t k,
                              void *stream) {
  clear_error();
  return gemm_fwd_groups(x, ws, ns, ys, count, m, k, as_stream(stream));
}

int32_t nf4s_gemm_fwd_grouped_ws(const uint16_t *x, const nf4s_tensor *ws, const int64_t *ns,
                                 uint16_t *const *ys, int32_t count, int64_t m, int64_t k,
                                 void *workspace, int64_t workspace_bytes, void *stream) {
  clear_error();
  if (workspace_bytes < 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "negative workspace size %lld",
                (long long)workspace_bytes);
  if (workspace != nullptr && !aligned(workspace, 16))
    return fail(NF4S_ERR_MISALIGNED, "workspace must be 16-byte aligned");
  return gemm_fwd_groups(x, ws, ns, ys, count, m, k, as_stream(stream), workspace,
                         workspace_bytes);
}

int32_t nf4s_gemm_fwd_workspace_size(const int64_t *ns, int32_t count, int64_t m, int64_t k,
                                     int64_t *bytes) {
  clear_error();
  return fwd_workspace_query(ns, count, m, k, bytes);
}

int32_t nf4s_gemm_fwd_swiglu(const uint16_t *x, const nf4s_tensor *w_gate,
                             const nf4s_tensor *w_up, int64_t m, int64_t ff, int64_t k,
                             uint16_t *hidden, void *stream) {
  clear_error();
  return gemm_swiglu(x, w_gate, w_up, m, ff, k, hidden, as_stream(stream));
}

int32_t nf4s_gemm_dgrad_sum(const uint16_t *const *dys, const nf4s_tensor *ws, const int64_t *ns,
                            int32_t count, int64_t m, int64_t k, uint16_t *dx, void *stream) {
  clear_error();
  return gemm_dgrad_groups(dys, ws, ns, count, m, k, dx, as_stream(stream));
}

int32_t nf4s_gemm_dgrad_sum_ws(const uint16_t *const *dys, const nf4s_tensor *ws,
                               const int64_t *ns, int32_t count, int64_t m, int64_t k,
                               uint16_t *dx, void *workspace, int64_t workspace_bytes,
                               void *stream) {
  clear_error();
  if (workspace_bytes < 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "negative workspace size %lld",
                (long long)workspace_bytes);
  if (workspace != nullptr && !aligned(workspace, 16))
    return fail(NF4S_ERR_MISALIGNED, "workspace must be 16-byte aligned");
  return gemm_dgrad_groups(dys, ws, ns, count, m, k, dx, as_stream(stream), workspace,
                           workspace_bytes);
}

int32_t nf4s_gemm_dgrad_workspace_size(const int64_t *ns, int32_t count, int64_t m, int64_t k,
                                       int64_t *bytes) {
  clear_error();
  if (bytes == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bytes is NULL");
  *bytes = 0;
  if (count <= 0 || count > kMaxGroups || ns == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "count must be 1..%d with sizes", kMaxGroups);
  *bytes = dgrad_workspace_bytes(ns, count, m, k);
  return NF4S_OK;
}

}  // extern "C"
