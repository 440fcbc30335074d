// nf4_codec.hip - NF4 quantize, double-quant encode and dequant kernels for
// gfx950, with their extern "C" entry points.
//
// Dequant is HBM-bound (2.52 B per element with double-quant, bf16 out): the
// fast kernel moves 16 B of packed nibbles per thread per chunk (32 elements),
// builds the 16-entry product table of the chunk's block in registers and
// writes 64 B of output with 128-bit non-temporal stores.  Anything the fast
// kernel cannot take (block size not a multiple of 32, unaligned pointers,
// the last n % 32 elements) goes through the element-wise kernel, which
// computes the same fp32 product and conversion.
#include "abi_common.hpp"
#include "nf4_device.hpp"

namespace nf4s {

__constant__ uint32_t kCodeTable[16] = {
    0xbf800000u, 0xbf3239b1u, 0xbf066b30u, 0xbeca32a0u,
    0xbe91a24du, 0xbe3d353fu, 0xbdba7872u, 0x00000000u,
    0x3da2faffu, 0x3e24cae3u, 0x3e7c04ddu, 0x3ead033au,
    0x3ee1a4b8u, 0x3f1007abu, 0x3f3913b3u, 0x3f800000u,
};

__device__ __forceinline__ float code_dyn(int i) {
  return __builtin_bit_cast(float, kCodeTable[i]);
}

// ---------------------------------------------------------------------------
// Quantize (shard_engine/python/pipeline/quantizer.py:21-53)
// ---------------------------------------------------------------------------

// NaN-propagating max, as torch's max(dim) over |x| (quantizer.py:35).
__device__ __forceinline__ float max_nan(float a, float b) {
  if (a != a) return a;
  if (b != b) return b;
  return b > a ? b : a;
}

// First-index argmin of |n - code_i| (quantizer.py:40-41) through the
// bracketing pair: j = last code <= n, then j or j+1 by the same fp32
// distances, j on ties.  Equal to the 16-way argmin for every fp32 n in
// [-1, 1] (checked exhaustively against the literal form on the CPU).
__device__ __forceinline__ uint32_t nf4_code(float n) {
  int j = 0;
#pragma unroll
  for (int i = 1; i < 16; ++i) j += (n >= code_value(i)) ? 1 : 0;
  if (n != n) return 0;  // torch argmin over an all-NaN row yields index 0
  if (j == 15) return 15;
  const float dl = fabsf(n - code_dyn(j));
  const float dr = fabsf(n - code_dyn(j + 1));
  return dr < dl ? (uint32_t)(j + 1) : (uint32_t)j;
}

// Element e of the input: fp32, or bf16 widened exactly (the bf16 weights a
// bf16 update leaves, doublepass/src/precision.rs:187-202).
template <typename T>
__device__ __forceinline__ float load_elem(const T *x, int64_t e);
template <>
__device__ __forceinline__ float load_elem<float>(const float *x, int64_t e) {
  return x[e];
}
template <>
__device__ __forceinline__ float load_elem<uint16_t>(const uint16_t *x, int64_t e) {
  return __builtin_bit_cast(float, (uint32_t)x[e] << 16);
}

// ---- Block-64 quantize: 8 elements per lane, 8 lanes per block ----------
//
// The code rule above is monotone in n (within a bracket the rounded
// distance to the lower code only grows and to the upper one only shrinks),
// so it is a step function of the fp32 quotient: code(n) = #{k : n >= S_k}
// for the 15 fp32 thresholds below (the smallest fp32 n with code(n) >= k;
// aethelstream_amd/code_steps.py derives them from the codebook, and an
// exhaustive CPU check over every fp32 in [-1, 1] compares the step form with
// the 16-way argmin).
__constant__ uint32_t kStepBits[15] = {
    0xbf591cd8u, 0xbf1c5270u, 0xbeeb847fu, 0xbeadea76u, 0xbe703cecu,
    0xbe0d38bbu, 0xbd3a7871u, 0x3d22fb00u, 0x3df64863u, 0x3e5067e1u,
    0x3e9582d5u, 0x3ec753fau, 0x3f006d04u, 0x3f248db0u, 0x3f5c89dau,
};

// Lookup: bucket i covers q in [-1 + i/16, -1 + (i+1)/16), i = 0 .. 32
// (bucket 32 is q = 1).  Consecutive steps are >= 0.08 apart, so a bucket
// holds at most one; entry i = {that step's bits (+inf if none), number of
// steps below the bucket}, and the code is base + (q >= step).
// The bucket comes from f = RN(q + 98304): f's ulp is 2^-7, so the low 11
// bits of f's pattern hold round(128 q) mod 2048, and those bits with the
// low 3 cleared are 8 (i - 16) mod 2048, the byte address of entry i in a
// 2 KB table.  Rounding moves q by <= 2^-8 and never down across an edge
// (edges are multiples of 2^-7); up across one only from q within 2^-8 below
// it, and no step lies within 0.0047 below an edge, so the entry counts the
// same steps as q's own bucket.
constexpr int kBuckets = 33;
constexpr int kStepTableWords = 256;  // 2 KB of uint2, 33 entries used

__device__ __forceinline__ void init_step_table(uint2 *tab) {
  const int i = (int)threadIdx.x;
  if (i < kBuckets) {
    const float lo = -1.0f + 0.0625f * (float)i, hi = lo + 0.0625f;
    uint32_t base = 0, step = 0x7f800000u;
#pragma unroll
    for (int k = 0; k < 15; ++k) {
      const float t = __builtin_bit_cast(float, kStepBits[k]);
      base += (t < lo) ? 1u : 0u;
      if (t >= lo && t < hi) step = kStepBits[k];
    }
    tab[(i - 16) & (kStepTableWords - 1)] = make_uint2(step, base);
  }
}

// Fast quotients q' = v * rcp(s) (v_rcp_f32, documented to 1 ulp; s in
// [1e-8, 2^126), so rcp(s) is a normal number) are within |q| 2^-23 (rcp's
// error) + 2^-25 (the product's rounding) < 2^-22 of v / s for |q| <= 1, and
// the exact RN(v / s) is within 2^-25 of v / s: q' and RN(v / s) can only
// fall on different sides of a step lying within 2^-21 of q'.  A lane with
// any q' within kMargin (twice that) of its bucket's step takes the exact
// quotient for all 8 elements (the bucket's step is the only one within
// 0.0016 of q').
constexpr float kMargin = 0x1p-20f;

// q in [-1 - 2^-8, 1 + 2^-8]; a NaN q reads some entry of the 2 KB table and
// its code is never used (its lane takes the exact path).
__device__ __forceinline__ uint32_t step_code(const uint2 *tab, float q, bool &near) {
  const float f = q + 98304.0f;
  const uint32_t addr = __builtin_bit_cast(uint32_t, f) & 0x7f8u;
  const uint2 t = *(const uint2 *)((const char *)tab + addr);
  const float step = __builtin_bit_cast(float, t.x);
  near |= fabsf(q - step) <= kMargin;
  return t.y + ((q >= step) ? 1u : 0u);
}

// The lane's 8 elements e0 .. e0+7 (all below the limit): 16-byte loads.
template <typename T>
__device__ __forceinline__ void load8_full(const T *__restrict__ x, int64_t e0, float v[8]) {
  // Elements go through scalar temporaries: hipcc folds a bit_cast of a
  // vector-element subscript to element 0 for every index.
  if constexpr (sizeof(T) == 4) {
    const u32x4 a = *(const u32x4 *)(x + e0);
    const u32x4 b = *(const u32x4 *)(x + e0 + 4);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t ak = a[k], bk = b[k];
      v[k] = __builtin_bit_cast(float, ak);
      v[4 + k] = __builtin_bit_cast(float, bk);
    }
  } else {
    const u32x4 a = *(const u32x4 *)(x + e0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t ak = a[k];
      v[2 * k] = __builtin_bit_cast(float, ak << 16);
      v[2 * k + 1] = __builtin_bit_cast(float, ak & 0xffff0000u);
    }
  }
}

// The lane's 8 elements, each loaded on its own, zero past `lim`
// (quantizer.py:30-32): any alignment, any tail.
template <typename T>
__device__ __forceinline__ void load8_guarded(const T *__restrict__ x, int64_t lim, int64_t e0,
                                              float v[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) v[k] = (e0 + k < lim) ? load_elem<T>(x, e0 + k) : 0.0f;
}

// Unsigned max of m and m of the lane that DPP control kCtrl names.
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_umax(uint32_t m) {
  const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, kCtrl, 0xF, 0xF, false);
  return (o > m) ? o : m;
}

// Codes of the lane's 8 elements, packed as quantizer.py:43-46 packs them
// (even element in the high nibble), and the block's unclamped absmax
// (:35, :48-53) in every lane of the block.  Call with the whole wave
// active: the absmax is reduced across the block's 8 lanes with DPP moves
// (quad xor 1, quad xor 2, half-row mirror) on the bit patterns of |x|,
// whose unsigned order is the numeric order with NaN above +inf (torch's
// max propagates NaN).
template <bool kFull>
__device__ __forceinline__ float encode8(const uint2 *tab, const float v[8], int64_t e0,
                                         int64_t lim, uint32_t &word) {
  float ml = __builtin_elementwise_maximum(fabsf(v[0]), fabsf(v[1]));  // NaN-propagating
#pragma unroll
  for (int k = 2; k < 8; ++k) ml = __builtin_elementwise_maximum(ml, fabsf(v[k]));
  uint32_t mb = __builtin_bit_cast(uint32_t, ml);
  mb = dpp_umax<0xB1>(mb);   // quad_perm [1,0,3,2]
  mb = dpp_umax<0x4E>(mb);   // quad_perm [2,3,0,1]
  mb = dpp_umax<0x141>(mb);  // row_half_mirror: lane i <-> 7-i within 8
  const float m = __builtin_bit_cast(float, mb);
  uint32_t c[8];
  // NaN, inf and absmax >= 2^126 (rcp would be subnormal) take the exact path.
  bool near = !(m < 0x1p126f);
  const float y = __builtin_amdgcn_rcpf(fmaxf(m, 1e-8f));
#pragma unroll
  for (int k = 0; k < 8; ++k) c[k] = step_code(tab, v[k] * y, near);
  if (near) {  // rare: the correctly rounded quotient, :36-38
    const float s = (m < 1e-8f) ? 1e-8f : m;  // clamp(min=1e-8); NaN stays NaN
    bool unused = false;
#pragma unroll
    for (int k = 0; k < 8; ++k) c[k] = step_code(tab, fmaxf(v[k] / s, -1.0f), unused);
  }
  if (!kFull && e0 + 8 > lim) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (e0 + k >= lim) c[k] = 0;  // odd-count pad nibble, :44-45
  }
  word = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) word |= ((c[2 * j] << 4) | c[2 * j + 1]) << (8 * j);
  return m;
}

// A tile is 8 blocks (512 elements) by one wave; lane l holds elements
// 8l .. 8l+7 of it, so the wave reads 2 KB (fp32) and writes 256 B
// contiguously.  tile_e0(t) is the first element of tile t and
// absmax_out(t, j, m) takes block j of tile t.

// One tile with every access guarded: elements at or past `lim` read as
// absent and are not written (the last, partial tile; unaligned buffers).
template <typename T, typename AbsmaxOut>
__device__ __forceinline__ void quantize_tile_guarded(const T *__restrict__ x, int64_t lim,
                                                      int64_t t, int64_t tile_e0,
                                                      const uint2 *tab,
                                                      uint8_t *__restrict__ packed,
                                                      AbsmaxOut absmax_out) {
  const int lane = threadIdx.x & 63;
  const int64_t e0 = tile_e0 + 8 * lane;
  float v[8];
  load8_guarded<T>(x, lim, e0, v);
  uint32_t word;
  const float m = encode8<false>(tab, v, e0, lim, word);
  if (e0 < lim) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (e0 + 2 * j < lim) packed[(e0 >> 1) + j] = (uint8_t)(word >> (8 * j));
    if ((lane & 7) == 0) absmax_out(t, lane >> 3, m);
  }
}

// Chunks of kU full tiles (x 16-byte and packed 4-byte aligned): one wave
// takes chunks c0, c0 + dc, ... < nchunks, with the next chunk's loads
// issued before the current chunk's codes (two register sets, alternating).
// Every path through a chunk issues the same loads and stores (all 8 lanes
// of a block store its absmax, the same value to the same address; the
// loop's exits each get their own copy of the codes), so the wait before a
// chunk's codes leaves the next chunk's loads and the last stores in flight.
template <typename T, int kU, typename TileE0, typename AbsmaxOut>
__device__ __forceinline__ void quantize_wave_full(const T *__restrict__ x, int64_t nchunks,
                                                   int64_t c0, int64_t dc, const uint2 *tab,
                                                   uint8_t *__restrict__ packed, TileE0 tile_e0,
                                                   AbsmaxOut absmax_out) {
  const int lane = threadIdx.x & 63;
  if (c0 >= nchunks) return;  // wave-uniform
  float va[kU][8], vb[kU][8];
  auto load = [&](float (&v)[kU][8], int64_t c) {
#pragma unroll
    for (int u = 0; u < kU; ++u) load8_full<T>(x, tile_e0(c * kU + u) + 8 * lane, v[u]);
  };
  auto emit = [&](float (&v)[kU][8], int64_t c) {
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int64_t t = c * kU + u;
      const int64_t e0 = tile_e0(t) + 8 * lane;
      uint32_t word;
      const float m = encode8<true>(tab, v[u], e0, 0, word);
      *(uint32_t *)(packed + (e0 >> 1)) = word;
      absmax_out(t, lane >> 3, m);
    }
  };
  load(va, c0);
  for (int64_t c = c0;;) {
    const int64_t cb = c + dc;
    if (cb >= nchunks) {  // wave-uniform
      emit(va, c);
      break;
    }
    load(vb, cb);
    emit(va, c);
    const int64_t ca = cb + dc;
    if (ca >= nchunks) {
      emit(vb, cb);
      break;
    }
    load(va, ca);
    emit(vb, cb);
    c = ca;
  }
}

// Tiles 0 .. ntiles-1 of a range whose elements end at `lim`, by wave `wid`
// of `nw`: whole chunks of full tiles through the pipelined path when kVec,
// the rest (the partial last tile, full tiles short of a chunk, every tile
// when !kVec) guarded.
template <typename T, bool kVec, int kU, typename TileE0, typename AbsmaxOut>
__device__ __forceinline__ void quantize_range(const T *__restrict__ x, int64_t lim,
                                               int64_t ntiles, int64_t wid, int64_t nw,
                                               const uint2 *tab, uint8_t *__restrict__ packed,
                                               TileE0 tile_e0, AbsmaxOut absmax_out) {
  int64_t t0 = 0;
  if (kVec) {
    const int64_t nfull = (tile_e0(ntiles - 1) + 512 <= lim) ? ntiles : ntiles - 1;
    const int64_t nchunks = nfull / kU;
    quantize_wave_full<T, kU>(x, nchunks, wid, nw, tab, packed, tile_e0, absmax_out);
    t0 = nchunks * kU;
  }
  for (int64_t t = t0 + wid; t < ntiles; t += nw)
    quantize_tile_guarded<T>(x, lim, t, tile_e0(t), tab, packed, absmax_out);
}

// kVec: x 16-byte and packed 4-byte aligned (16-byte loads, 4-byte stores).
template <typename T, bool kVec, int kU>
__global__ void __launch_bounds__(256) quantize64_kernel(const T *__restrict__ x, int64_t n,
                                                         uint8_t *__restrict__ packed,
                                                         float *__restrict__ absmax,
                                                         int64_t ntiles) {
  __shared__ uint2 tab[kStepTableWords];
  init_step_table(tab);
  __syncthreads();
  quantize_range<T, kVec, kU>(
      x, n, ntiles, (int64_t)blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6),
      (int64_t)gridDim.x * 4, tab,
      packed, [](int64_t t) { return t * 512; },
      [=](int64_t t, int j, float m) { absmax[t * 8 + j] = m; });  // :48-53, unclamped
}

// Any block size: per-block absmax, then per-byte codes.
__global__ void absmax_generic_kernel(const float *__restrict__ x, int64_t n, int32_t bs,
                                      float *__restrict__ absmax, int64_t nblocks) {
  for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nblocks;
       b += (int64_t)gridDim.x * blockDim.x) {
    float m = 0.0f;
    const int64_t s = b * bs;
    for (int64_t i = s; i < s + bs && i < n; ++i) m = max_nan(m, fabsf(x[i]));
    absmax[b] = m;
  }
}

__global__ void codes_generic_kernel(const float *__restrict__ x, int64_t n, int32_t bs,
                                     const float *__restrict__ absmax,
                                     uint8_t *__restrict__ packed, int64_t npacked) {
  for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < npacked;
       j += (int64_t)gridDim.x * blockDim.x) {
    uint32_t byte = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int64_t e = 2 * j + h;
      uint32_t c = 0;
      if (e < n) {
        const float m = absmax[e / bs];
        const float safe = (m < 1e-8f) ? 1e-8f : m;
        c = nf4_code(x[e] / safe);
      }
      byte |= c << (h ? 0 : 4);
    }
    packed[j] = (uint8_t)byte;
  }
}

// ---------------------------------------------------------------------------
// Double-quant encode (conventions of galore/src/quantize.rs:4-13)
// ---------------------------------------------------------------------------

// Scale of a double-quant group from its largest absmax (1.0 for an all-zero
// group, galore/src/quantize.rs:8-12), and the code of one absmax: round
// half to even, clamped to 0..127 (NaN -> 0).
__device__ __forceinline__ float dq_scale(float mx) { return (mx <= 0.0f) ? 1.0f : mx / 127.0f; }
__device__ __forceinline__ uint8_t dq_code(float a, float sc) {
  float r = rintf(a / sc);  // round half to even
  if (!(r >= 0.0f)) r = 0.0f;
  if (r > 127.0f) r = 127.0f;
  return (uint8_t)r;
}

__global__ void __launch_bounds__(256) dq_encode_kernel(const float *__restrict__ absmax,
                                                        int64_t nblocks, int32_t group,
                                                        uint8_t *__restrict__ q,
                                                        float *__restrict__ scale) {
  __shared__ float red[4];
  const int64_t g = blockIdx.x;
  const int64_t s = g * group;
  const int64_t e = (s + group < nblocks) ? s + group : nblocks;
  float m = 0.0f;
  for (int64_t i = s + threadIdx.x; i < e; i += blockDim.x) {
    const float a = absmax[i];
    m = (a > m) ? a : m;  // NaN never wins, as in the CPU encode
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(m, off, 64);
    m = (o > m) ? o : m;
  }
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float mx = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) mx = (red[w] > mx) ? red[w] : mx;
  const float sc = dq_scale(mx);
  if (threadIdx.x == 0) scale[g] = sc;
  for (int64_t i = s + threadIdx.x; i < e; i += blockDim.x) q[i] = dq_code(absmax[i], sc);
}

// Quantize + double-quant in one pass, for weights re-quantized on the device
// after an update (FlowCast::on_weights_updated, flowcast/src/lib.rs:501-521,
// after apply_galore_bf16_update, doublepass/src/precision.rs:187-202): each
// workgroup takes groups of `group` 64-element blocks in turn (a grid of at
// most kQuantMaxGrid), its waves taking a group's 8-block tiles in turn (the
// same lane code as quantize64_kernel).
// The block absmax stay in LDS (never written as fp32), so the call needs no
// scratch memory; codes come from the fp32 absmax exactly as quantize64_kernel
// computes them, and q / scale exactly as dq_encode_kernel does.
template <typename T, bool kVec, int kU>
__global__ void __launch_bounds__(256) quantize_dq_kernel(const T *__restrict__ x, int64_t n,
                                                          int32_t group,
                                                          uint8_t *__restrict__ packed,
                                                          uint8_t *__restrict__ q,
                                                          float *__restrict__ scale,
                                                          int64_t nblocks, int64_t ngroups) {
  extern __shared__ float am_lds[];  // `group` block absmax
  __shared__ uint2 tab[kStepTableWords];
  __shared__ float red[4];
  init_step_table(tab);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // Persistent: workgroup b takes groups b, b + grid, ...
  for (int64_t grp = blockIdx.x; grp < ngroups; grp += gridDim.x) {
    const int64_t b0 = grp * group;
    const int64_t nb = (b0 + group < nblocks) ? group : nblocks - b0;
    // Elements of this group's blocks: the others read as absent, so a tile
    // that runs past the group (group < 8) neither counts nor writes them.
    const int64_t lim = (64 * (b0 + nb) < n) ? 64 * (b0 + nb) : n;
    quantize_range<T, kVec, kU>(
        x, lim, (nb + 7) >> 3, __builtin_amdgcn_readfirstlane(wave), 4, tab, packed,
        [=](int64_t t) { return (b0 + 8 * t) * 64; },
        [=](int64_t t, int j, float m) { am_lds[8 * t + j] = m; });
    __syncthreads();
    float m = 0.0f;
    for (int64_t i = threadIdx.x; i < nb; i += blockDim.x) {
      const float a = am_lds[i];
      m = (a > m) ? a : m;  // NaN never wins, as in dq_encode_kernel
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float o = __shfl_xor(m, off, 64);
      m = (o > m) ? o : m;
    }
    if (lane == 0) red[wave] = m;
    __syncthreads();
    float mx = red[0];
    for (int w = 1; w < 4; ++w) mx = (red[w] > mx) ? red[w] : mx;
    const float sc = dq_scale(mx);
    if (threadIdx.x == 0) scale[grp] = sc;
    for (int64_t i = threadIdx.x; i < nb; i += blockDim.x) q[b0 + i] = dq_code(am_lds[i], sc);
    // The next group's absmax and partial maxima overwrite am_lds and red.
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Dequant (shard_engine/src/nf4.rs:37-83)
// ---------------------------------------------------------------------------

constexpr int kMaxBatch = 16;
constexpr int32_t kMaxDqGroup = 8192;  // quantize_dq_kernel keeps a group's absmax in LDS
constexpr int kDqWaves = 2;                        // waves per workgroup
constexpr int kDqThreads = 64 * kDqWaves;
constexpr int64_t kTileChunks = 64 * kDqWaves;     // one 32-element chunk per lane

struct DqEntry {
  const uint8_t *packed;
  AbsmaxRef am;
  int32_t block_size;
  uint16_t *out;
  int64_t nchunks;     // full 32-element chunks handled here
  int64_t tile_begin;  // first tile index of this entry in the launch
};

struct DqBatch {
  DqEntry e[kMaxBatch];
  int32_t count;
};

// One chunk = 32 elements = 16 B of packed nibbles -> 64 B of output, all in
// one absmax block (block_size % 32 == 0).  Each wave takes 64 consecutive
// chunks: each lane loads one 16-B chunk (a coalesced 1 KB per wave), builds
// that block's product table and dequantizes into LDS, and the wave then
// writes its 4 KB of output as four contiguous 1 KB stores.  Scattered 16-B
// stores at a 64-B stride measured 7x slower on MI355X than these contiguous
// ones.
// Small one-shot workgroups (2 waves, 8 KB of output, consecutive workgroups
// on consecutive XCDs) keep the HBM write stream fastest: on MI355X this
// shape measured 6.13 TB/s against 5.75 TB/s for 4-wave workgroups whose
// waves each dequantized two rounds (32 KB per workgroup), and a write-only
// fill shows the same preference (6.5 TB/s at 4 KB per workgroup, 5.3 TB/s
// at 64 KB).
// Cache policy: the packed nibbles load with the default policy (a
// non-temporal load measured 6.13-6.32 TB/s against 6.83-6.85), and the
// output goes out non-temporal and sc1 (kStoreNtSc1; 6.89-6.91 TB/s, nt
// alone 6.83-6.85, the default policy 5.77-5.79).  The same access pattern
// without the lookup work measured 6.90-6.91 TB/s: the lookup is hidden.
// Buffer-instruction cache-policy bits on gfx950: nt (bit 1) | sc1 (bit 4).
constexpr int kStoreNtSc1 = 2 | 16;

template <bool kF16>
__global__ void __launch_bounds__(kDqThreads) dequant_fast_kernel(const DqBatch batch) {
  __shared__ u32x4 stage[kDqWaves][64 * 4 + 4];  // per wave 4 KB, +1 pad unit per 16 lanes
  const int64_t tile = blockIdx.x;
  int idx = 0;
#pragma unroll 1
  for (int i = 1; i < batch.count; ++i)
    if (tile >= batch.e[i].tile_begin) idx = i;
  const DqEntry &E = batch.e[idx];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int64_t cbase = (tile - E.tile_begin) * kTileChunks + wave * 64;
  const int64_t nchunks = E.nchunks;
  if (cbase >= nchunks) return;  // wave-uniform
  const u32x4 *src = reinterpret_cast<const u32x4 *>(E.packed);
  // The wave's 64 chunks of output (4 KB) through a buffer resource, for the
  // store's cache-policy bits; its size also bounds the stores.
  const int64_t units = (nchunks - cbase < 64 ? nchunks - cbase : 64) * 4;
  const __amdgpu_buffer_rsrc_t dst = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(E.out + cbase * 32), 0, (int)(units * 16), 0x00020000);
  const int64_t c = cbase + lane;
  if (c < nchunks) {
    const u32x4 w = src[c];
    const Lut16 lut = make_lut<kF16>(load_absmax(E.am, (c * 32) / E.block_size));
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint32_t o[4];
      lut_apply8(lut, words[k], o);
      u32x4 v;
      v.x = o[0]; v.y = o[1]; v.z = o[2]; v.w = o[3];
      const int u = lane * 4 + k;  // 16-B unit of the wave's 4 KB
      stage[wave][u + (u >> 6)] = v;
    }
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int u = k * 64 + lane;
    if (u < units) {
      typedef unsigned int uvec4 __attribute__((ext_vector_type(4)));
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(uvec4, stage[wave][u + (u >> 6)]), dst, u * 16, 0, kStoreNtSc1);
    }
  }
}

template <bool kF16>
__global__ void dequant_elem_kernel(const uint8_t *__restrict__ packed, AbsmaxRef am,
                                    int32_t bs, uint16_t *__restrict__ out, int64_t begin,
                                    int64_t end) {
  for (int64_t e = begin + (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < end;
       e += (int64_t)gridDim.x * blockDim.x) {
    const uint32_t byte = packed[e >> 1];
    const uint32_t nib = (e & 1) ? (byte & 15u) : (byte >> 4);
    const float v = fp32_rounded(code_dyn((int)nib) * load_absmax(am, e / bs));
    uint16_t r;
    if (kF16) r = __builtin_bit_cast(uint16_t, (_Float16)v);
    else r = __builtin_bit_cast(uint16_t, (__bf16)v);
    out[e] = r;
  }
}

static AbsmaxRef absmax_ref(const nf4s_tensor &t) {
  AbsmaxRef a;
  a.absmax = t.absmax;
  a.q = t.absmax_q;
  a.scale = t.absmax_scale;
  a.group_shift = t.dq_group > 0 ? group_shift(t.dq_group) : 0;
  a.block_shift = 0;  // the GEMMs' field; the dequant kernels index by block_size
  return a;
}

static bool fast_ok(const nf4s_tensor &t, const uint16_t *out) {
  return t.block_size % 32 == 0 && aligned(t.packed, 16) && aligned(out, 16);
}

static int grid_for(int64_t work, int threads) {
  int64_t g = (work + threads - 1) / threads;
  if (g > 65536) g = 65536;
  return (int)(g < 1 ? 1 : g);
}

template <bool kF16>
static int32_t dequant_batch(const nf4s_tensor *ts, const int64_t *ns, uint16_t *const *outs,
                             int32_t count, hipStream_t stream) {
  if (count < 0 || count > kMaxBatch)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "batch count %d outside [0, %d]", count, kMaxBatch);
  if (count > 0 && (ts == nullptr || ns == nullptr || outs == nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "batch arrays are NULL");
  for (int i = 0; i < count; ++i) {
    const int32_t rc = validate_tensor(&ts[i], ns[i]);
    if (rc != NF4S_OK) return rc;
    if (ns[i] > 0 && outs[i] == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "output is NULL");
  }
  DqBatch batch{};
  int64_t tiles = 0;
  for (int i = 0; i < count; ++i) {
    const nf4s_tensor &t = ts[i];
    const int64_t n = ns[i];
    const bool fast = fast_ok(t, outs[i]);
    const int64_t nchunks = fast ? n / 32 : 0;
    if (nchunks > 0) {
      DqEntry &E = batch.e[batch.count++];
      E.packed = t.packed;
      E.am = absmax_ref(t);
      E.block_size = t.block_size;
      E.out = outs[i];
      E.nchunks = nchunks;
      E.tile_begin = tiles;
      tiles += (nchunks + kTileChunks - 1) / kTileChunks;
    }
    const int64_t tail_begin = nchunks * 32;
    if (tail_begin < n) {
      hipLaunchKernelGGL(dequant_elem_kernel<kF16>, dim3(grid_for(n - tail_begin, 256)),
                         dim3(256), 0, stream, t.packed, absmax_ref(t), t.block_size, outs[i],
                         tail_begin, n);
      const int32_t rc = check_launch("dequant_elem_kernel");
      if (rc != NF4S_OK) return rc;
    }
  }
  if (tiles > 0) {
    if (tiles > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many tiles");
    hipLaunchKernelGGL(dequant_fast_kernel<kF16>, dim3((uint32_t)tiles), dim3(kDqThreads), 0,
                       stream, batch);
    return check_launch("dequant_fast_kernel");
  }
  return NF4S_OK;
}

constexpr int kQuantU = 1;         // tiles per chunk
constexpr int kQuantMaxGrid = 1024;  // workgroups of the block-64 quantize launches

template <typename T>
static bool quantize_vec_ok(const T *x, const uint8_t *packed) {
  return ((uintptr_t)x % 16 == 0) && ((uintptr_t)packed % 4 == 0);
}

template <typename T>
static int32_t quantize64(const T *x, int64_t n, uint8_t *packed, float *absmax, hipStream_t s) {
  const int64_t ntiles = ceil_div(n, 512);
  int64_t grid = ((ntiles + kQuantU - 1) / kQuantU + 3) / 4;
  if (grid > kQuantMaxGrid) grid = kQuantMaxGrid;
  if (quantize_vec_ok(x, packed))
    hipLaunchKernelGGL((quantize64_kernel<T, true, kQuantU>), dim3((uint32_t)grid), dim3(256), 0, s, x, n,
                       packed, absmax, ntiles);
  else
    hipLaunchKernelGGL((quantize64_kernel<T, false, kQuantU>), dim3((uint32_t)grid), dim3(256), 0, s, x, n,
                       packed, absmax, ntiles);
  return check_launch("quantize64_kernel");
}

template <typename T>
static int32_t quantize_dq(const T *x, int64_t n, int32_t block_size, int32_t group,
                           uint8_t *packed, uint8_t *q, float *scale, void *stream) {
  if (n < 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "negative element count");
  if (block_size != 64)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "quantize + double-quant needs block_size 64, got %d",
                block_size);
  if (group <= 0 || (group & (group - 1)) != 0 || group > kMaxDqGroup)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "group must be a power of two <= %d, got %d",
                kMaxDqGroup, group);
  if (n == 0) return NF4S_OK;
  if (x == nullptr || packed == nullptr || q == nullptr || scale == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL buffer");
  const int64_t nb = ceil_div(n, 64);
  const int64_t ng = ceil_div(nb, group);
  if (ng > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many groups");
  const size_t lds = (size_t)group * sizeof(float);
  const uint32_t grid = (uint32_t)(ng < kQuantMaxGrid ? ng : kQuantMaxGrid);
  if (quantize_vec_ok(x, packed))
    hipLaunchKernelGGL((quantize_dq_kernel<T, true, kQuantU>), dim3(grid), dim3(256), lds,
                       as_stream(stream), x, n, group, packed, q, scale, nb, ng);
  else
    hipLaunchKernelGGL((quantize_dq_kernel<T, false, kQuantU>), dim3(grid), dim3(256), lds,
                       as_stream(stream), x, n, group, packed, q, scale, nb, ng);
  return check_launch("quantize_dq_kernel");
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

int32_t nf4s_quantize(const float *x, int64_t n, int32_t block_size, uint8_t *packed,
                      float *absmax, void *stream) {
  clear_error();
  if (n < 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "negative element count");
  if (block_size <= 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "block_size must be positive");
  if (n == 0) return NF4S_OK;
  if (x == nullptr || packed == nullptr || absmax == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL buffer");
  const int64_t nb = ceil_div(n, block_size);
  hipStream_t s = as_stream(stream);
  if (block_size == 64) return quantize64<float>(x, n, packed, absmax, s);
  hipLaunchKernelGGL(absmax_generic_kernel, dim3(grid_for(nb, 256)), dim3(256), 0, s, x, n,
                     block_size, absmax, nb);
  int32_t rc = check_launch("absmax_generic_kernel");
  if (rc != NF4S_OK) return rc;
  const int64_t npk = ceil_div(n, 2);
  hipLaunchKernelGGL(codes_generic_kernel, dim3(grid_for(npk, 256)), dim3(256), 0, s, x, n,
                     block_size, absmax, packed, npk);
  return check_launch("codes_generic_kernel");
}

int32_t nf4s_quantize_bf16(const uint16_t *x, int64_t n, int32_t block_size, uint8_t *packed,
                           float *absmax, void *stream) {
  clear_error();
  if (n < 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "negative element count");
  if (block_size != 64)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "bf16 quantize needs block_size 64, got %d",
                block_size);
  if (n == 0) return NF4S_OK;
  if (x == nullptr || packed == nullptr || absmax == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL buffer");
  return quantize64<uint16_t>(x, n, packed, absmax, as_stream(stream));
}

int32_t nf4s_quantize_dq(const float *x, int64_t n, int32_t block_size, int32_t group,
                         uint8_t *packed, uint8_t *absmax_q, float *absmax_scale, void *stream) {
  clear_error();
  return quantize_dq<float>(x, n, block_size, group, packed, absmax_q, absmax_scale, stream);
}

int32_t nf4s_quantize_dq_bf16(const uint16_t *x, int64_t n, int32_t block_size, int32_t group,
                              uint8_t *packed, uint8_t *absmax_q, float *absmax_scale,
                              void *stream) {
  clear_error();
  return quantize_dq<uint16_t>(x, n, block_size, group, packed, absmax_q, absmax_scale, stream);
}

int32_t nf4s_dq_encode(const float *absmax, int64_t nblocks, int32_t group, uint8_t *q,
                       float *scale, void *stream) {
  clear_error();
  if (nblocks < 0 || group <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "nblocks must be >= 0 and group > 0");
  if (nblocks == 0) return NF4S_OK;
  if (absmax == nullptr || q == nullptr || scale == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "NULL buffer");
  const int64_t ng = ceil_div(nblocks, group);
  if (ng > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many groups");
  hipLaunchKernelGGL(dq_encode_kernel, dim3((uint32_t)ng), dim3(256), 0, as_stream(stream),
                     absmax, nblocks, group, q, scale);
  return check_launch("dq_encode_kernel");
}

int32_t nf4s_dequant_f16(const nf4s_tensor *t, int64_t n, uint16_t *out, void *stream) {
  clear_error();
  if (t == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "tensor descriptor is NULL");
  uint16_t *outs[1] = {out};
  return dequant_batch<true>(t, &n, outs, 1, as_stream(stream));
}

int32_t nf4s_dequant_bf16(const nf4s_tensor *t, int64_t n, uint16_t *out, void *stream) {
  clear_error();
  if (t == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "tensor descriptor is NULL");
  uint16_t *outs[1] = {out};
  return dequant_batch<false>(t, &n, outs, 1, as_stream(stream));
}

int32_t nf4s_dequant_batch_bf16(const nf4s_tensor *ts, const int64_t *ns, uint16_t *const *outs,
                                int32_t count, void *stream) {
  clear_error();
  return dequant_batch<false>(ts, ns, outs, count, as_stream(stream));
}

}  // extern "C"
