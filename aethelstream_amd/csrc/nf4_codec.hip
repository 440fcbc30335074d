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

// One 64-element block by one wave, one lane per element: returns the block's
// unclamped absmax (in every lane) and writes its packed codes.
template <typename T>
__device__ __forceinline__ float quantize_block64(const T *__restrict__ x, int64_t n, int64_t b,
                                                  int lane, uint8_t *__restrict__ packed) {
  const int64_t e = b * 64 + lane;
  const float v = (e < n) ? load_elem<T>(x, e) : 0.0f;  // zero padding, quantizer.py:30-32
  float m = fabsf(v);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = max_nan(m, __shfl_xor(m, off, 64));
  const float safe = (m < 1e-8f) ? 1e-8f : m;          // clamp(min=1e-8), :36
  const float nv = v / safe;                           // correctly rounded, :38
  uint32_t c = nf4_code(nv);
  uint32_t c1 = __shfl_xor(c, 1, 64);
  if (e + 1 >= n) c1 = 0;                              // odd-count pad nibble, :44-45
  if ((lane & 1) == 0 && e < n) packed[e >> 1] = (uint8_t)((c << 4) | c1);  // :46
  return m;                                            // unclamped, :48-53
}

// block_size == 64: one wave per block.
template <typename T>
__global__ void __launch_bounds__(256) quantize64_kernel(const T *__restrict__ x, int64_t n,
                                                         uint8_t *__restrict__ packed,
                                                         float *__restrict__ absmax,
                                                         int64_t nblocks) {
  const int lane = threadIdx.x & 63;
  const int64_t wave0 = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int64_t nwaves = (int64_t)gridDim.x * (blockDim.x >> 6);
  for (int64_t b = wave0; b < nblocks; b += nwaves) {
    const float m = quantize_block64<T>(x, n, b, lane, packed);
    if (lane == 0) absmax[b] = m;
  }
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
// after apply_galore_bf16_update, doublepass/src/precision.rs:187-202): one
// workgroup per group of `group` 64-element blocks.
// The block absmax stay in LDS (never written as fp32), so the call needs no
// scratch memory; codes come from the fp32 absmax exactly as quantize64_kernel
// computes them, and q / scale exactly as dq_encode_kernel does.
template <typename T>
__global__ void __launch_bounds__(256) quantize_dq_kernel(const T *__restrict__ x, int64_t n,
                                                          int32_t group,
                                                          uint8_t *__restrict__ packed,
                                                          uint8_t *__restrict__ q,
                                                          float *__restrict__ scale,
                                                          int64_t nblocks) {
  extern __shared__ float am_lds[];  // `group` block absmax
  __shared__ float red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t b0 = (int64_t)blockIdx.x * group;
  const int64_t nb = (b0 + group < nblocks) ? group : nblocks - b0;
  for (int64_t i = wave; i < nb; i += 4) {
    const float m = quantize_block64<T>(x, n, b0 + i, lane, packed);
    if (lane == 0) am_lds[i] = m;
  }
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
  if (threadIdx.x == 0) scale[blockIdx.x] = sc;
  for (int64_t i = threadIdx.x; i < nb; i += blockDim.x) q[b0 + i] = dq_code(am_lds[i], sc);
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
  const int64_t nb = (n + 63) / 64;
  const int64_t ng = (nb + group - 1) / group;
  if (ng > 0x7fffffff) return fail(NF4S_ERR_UNSUPPORTED_SHAPE, "too many groups");
  hipLaunchKernelGGL(quantize_dq_kernel<T>, dim3((uint32_t)ng), dim3(256),
                     (size_t)group * sizeof(float), as_stream(stream), x, n, group, packed, q,
                     scale, nb);
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
  const int64_t nb = (n + block_size - 1) / block_size;
  hipStream_t s = as_stream(stream);
  if (block_size == 64) {
    const int64_t wg = (nb + 3) / 4;
    hipLaunchKernelGGL(quantize64_kernel<float>, dim3(grid_for(wg, 1)), dim3(256), 0, s, x, n,
                       packed, absmax, nb);
    return check_launch("quantize64_kernel");
  }
  hipLaunchKernelGGL(absmax_generic_kernel, dim3(grid_for(nb, 256)), dim3(256), 0, s, x, n,
                     block_size, absmax, nb);
  int32_t rc = check_launch("absmax_generic_kernel");
  if (rc != NF4S_OK) return rc;
  const int64_t npk = (n + 1) / 2;
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
  const int64_t nb = (n + 63) / 64;
  hipLaunchKernelGGL(quantize64_kernel<uint16_t>, dim3(grid_for((nb + 3) / 4, 1)), dim3(256), 0,
                     as_stream(stream), x, n, packed, absmax, nb);
  return check_launch("quantize64_kernel");
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
  const int64_t ng = (nblocks + group - 1) / group;
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
