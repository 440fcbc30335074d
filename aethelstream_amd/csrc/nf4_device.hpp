// nf4_device.hpp - device-side NF4 helpers shared by the codec and GEMM
// kernels (gfx950).
//
// The hot dequant step turns one 32-bit word of packed nibbles (8 elements)
// into four bf16x2 (or f16x2) words with a per-block product table held in
// registers and looked up with v_perm_b32 byte selects:
//   T[i] = cvt(code[i] * absmax)          16 products, one fp32 multiply each
// so every output is bit-identical to cvt(code * absmax) computed per element
// (shard_engine/src/nf4.rs:76-78): each product depends on (code, absmax) only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nf4s {

// Native clang vector types (usable with the nontemporal builtins).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// shard_engine/src/nf4.rs:6-23, as fp32 bit patterns.
__device__ constexpr uint32_t kCodeBits[16] = {
    0xbf800000u, 0xbf3239b1u, 0xbf066b30u, 0xbeca32a0u,
    0xbe91a24du, 0xbe3d353fu, 0xbdba7872u, 0x00000000u,
    0x3da2faffu, 0x3e24cae3u, 0x3e7c04ddu, 0x3ead033au,
    0x3ee1a4b8u, 0x3f1007abu, 0x3f3913b3u, 0x3f800000u,
};

__device__ __forceinline__ float code_value(int i) {
  return __builtin_bit_cast(float, kCodeBits[i]);
}

// The reference rounds twice: the fp32 product code * absmax, then the f16 /
// bf16 conversion (shard_engine/src/nf4.rs:77-78).  hipcc otherwise folds
// fptrunc(fmul) into one v_fma_mix* with a single rounding of the exact
// product (even under -ffp-contract=off), which differs on conversion ties.
// The empty asm hands the conversion an opaque, already-rounded fp32 value.
__device__ __forceinline__ float fp32_rounded(float x) {
  asm("" : "+v"(x));
  return x;
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// fp32 pair -> bf16 pair, round to nearest even: one v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, bf16x2_t));
}

// fp32 pair -> IEEE binary16 pair, round to nearest even: one v_cvt_pk_f16_f32.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){lo, hi}, f16x2_t));
}

__device__ __forceinline__ uint32_t perm(uint32_t hi4, uint32_t lo4, uint32_t sel) {
  // Result byte i = byte sel.byte[i] of the 8-byte value {hi4:lo4}.
  return __builtin_amdgcn_perm(hi4, lo4, sel);
}

// Byte-split product table: lo[t] holds the low bytes of entries 4t..4t+3,
// hi[t] their high bytes.
struct Lut16 {
  uint32_t lo[4];
  uint32_t hi[4];
};

template <bool kF16>
__device__ __forceinline__ Lut16 make_lut(float absmax) {
  uint32_t d[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float p0 = fp32_rounded(code_value(2 * j) * absmax);
    const float p1 = fp32_rounded(code_value(2 * j + 1) * absmax);
    d[j] = kF16 ? pack_f16x2(p0, p1) : pack_bf16x2(p0, p1);
  }
  Lut16 t;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    // d[2q] = {T[4q], T[4q+1]}, d[2q+1] = {T[4q+2], T[4q+3]}.
    t.lo[q] = perm(d[2 * q + 1], d[2 * q], 0x06040200u);
    t.hi[q] = perm(d[2 * q + 1], d[2 * q], 0x07050301u);
  }
  return t;
}

// 16-entry byte lookup: 3-bit index in each selector byte, bit 3 of the
// nibble given as a per-byte 0x00/0xff mask.
__device__ __forceinline__ uint32_t lookup16(const uint32_t tab[4], uint32_t sel,
                                             uint32_t mask) {
  const uint32_t a = perm(tab[1], tab[0], sel);  // entries 0..7
  const uint32_t b = perm(tab[3], tab[2], sel);  // entries 8..15
  return (b & mask) | (a & ~mask);
}

// The lookup of one packed word w (byte k holds element 2k in its high nibble
// and 2k+1 in its low nibble), split into stages so that a caller can spread
// them between other instructions:
//   word_select:  3-bit selectors and bit-3 masks of the even / odd nibbles
//   word_even:    low and high result bytes of the 4 even elements
//   word_odd:     low and high result bytes of the 4 odd elements
//   word_merge:   out[j] = elem 2j | elem 2j+1 << 16 (natural element order)
struct WordLookup {
  uint32_t selE, selO, maskE, maskO;
  uint32_t loE, hiE, loO, hiO;
};

// v_perm_b32 selector values 8, 9, 10 and 11 replicate the top bit of byte
// 1, 3, 5 and 7 of {hi4:lo4} into a whole byte.  With hi4 = v and
// lo4 = v << 8, bytes 1, 3, 5, 7 are bytes 0, 2, 1, 3 of v, so kSignBytes
// turns bit 7 of every byte of v into a 0x00 / 0xff byte mask.
constexpr uint32_t kSignBytes = 0x0B090A08u;

// word_select in two halves: the 3-bit selectors, then the bit-3 masks.
__device__ __forceinline__ void word_select_idx(uint32_t w, WordLookup &x) {
  x.selE = (w >> 4) & 0x07070707u;
  x.selO = w & 0x07070707u;
}

__device__ __forceinline__ void word_select_mask(uint32_t w, WordLookup &x) {
  x.maskE = perm(w, w << 8, kSignBytes);          // bit 3 of each high nibble
  x.maskO = perm(w << 4, w << 12, kSignBytes);    // bit 3 of each low nibble
}

__device__ __forceinline__ void word_select(uint32_t w, WordLookup &x) {
  word_select_idx(w, x);
  word_select_mask(w, x);
}

__device__ __forceinline__ void word_even(const Lut16 &t, WordLookup &x) {
  x.loE = lookup16(t.lo, x.selE, x.maskE);
  x.hiE = lookup16(t.hi, x.selE, x.maskE);
}

__device__ __forceinline__ void word_odd(const Lut16 &t, WordLookup &x) {
  x.loO = lookup16(t.lo, x.selO, x.maskO);
  x.hiO = lookup16(t.hi, x.selO, x.maskO);
}

// First half of the merge: whole 16-bit elements, pairs in the order
//   pairs[0] = elem0 | elem2 << 16    pairs[1] = elem1 | elem3 << 16
//   pairs[2] = elem4 | elem6 << 16    pairs[3] = elem5 | elem7 << 16
// so element j is half (j >> 1) & 1 of pairs[(j & 1) + 2 * (j >> 2)].
__device__ __forceinline__ void word_pairs(const WordLookup &x, uint32_t pairs[4]) {
  pairs[0] = perm(x.hiE, x.loE, 0x05010400u);
  pairs[1] = perm(x.hiO, x.loO, 0x05010400u);
  pairs[2] = perm(x.hiE, x.loE, 0x07030602u);
  pairs[3] = perm(x.hiO, x.loO, 0x07030602u);
}

// Second half of the merge: natural element order from word_pairs' output.
__device__ __forceinline__ void pairs_merge(const uint32_t p[4], uint32_t out[4]) {
  out[0] = perm(p[1], p[0], 0x05040100u);
  out[1] = perm(p[1], p[0], 0x07060302u);
  out[2] = perm(p[3], p[2], 0x05040100u);
  out[3] = perm(p[3], p[2], 0x07060302u);
}

__device__ __forceinline__ void word_merge(const WordLookup &x, uint32_t out[4]) {
  uint32_t p[4];
  word_pairs(x, p);
  pairs_merge(p, out);
}

// The GEMMs' lookup of one packed word, in memory order: elements 0-3 and
// 4-7 each get one selector word (the nibble of element i in byte i), so the
// byte-plane lookups already hold elements in order and one perm level
// interleaves the low and high planes into bf16 pairs (word_merge needs two).
// Bit 3 of a nibble picks the plane half through the last perm's selector
// (byte i + 4 * bit 3) instead of a byte mask.  25 VALU instructions per
// word against 28 for WordLookup.
struct NatLookup {
  uint32_t selA, selB;  // 3-bit selectors of elements 0-3 / 4-7
  uint32_t ctlA, ctlB;  // byte i: i + 4 * (bit 3 of the element's nibble)
  uint32_t loA, hiA, loB, hiB;
};

// Byte i of {w : w >> 4} at 4 + k is byte k of w (element 2k + 1 in its low
// nibble), at k byte k of w >> 4 (element 2k in its low nibble).
__device__ __forceinline__ void nat_select(uint32_t w, NatLookup &x) {
  const uint32_t t4 = w >> 4;
  x.selA = perm(w, t4, 0x05010400u);
  x.selB = perm(w, t4, 0x07030602u);
}

// (v & 0x04040404) | 0x03020100 in one instruction.
__device__ __forceinline__ uint32_t nat_ctl(uint32_t v) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(v), "s"(0x04040404u), "v"(0x03020100u));
  return r;
}

__device__ __forceinline__ void nat_controls(NatLookup &x) {
  x.ctlA = nat_ctl(x.selA >> 1);
  x.ctlB = nat_ctl(x.selB >> 1);
  x.selA &= 0x07070707u;
  x.selB &= 0x07070707u;
}

__device__ __forceinline__ uint32_t nat_lookup16(const uint32_t tab[4], uint32_t sel, uint32_t ctl) {
  return perm(perm(tab[3], tab[2], sel), perm(tab[1], tab[0], sel), ctl);
}

__device__ __forceinline__ void nat_planes_a(const Lut16 &t, NatLookup &x) {
  x.loA = nat_lookup16(t.lo, x.selA, x.ctlA);
  x.hiA = nat_lookup16(t.hi, x.selA, x.ctlA);
}

__device__ __forceinline__ void nat_planes_b(const Lut16 &t, NatLookup &x) {
  x.loB = nat_lookup16(t.lo, x.selB, x.ctlB);
  x.hiB = nat_lookup16(t.hi, x.selB, x.ctlB);
}

// out[j] = elem 2j | elem 2j+1 << 16.
__device__ __forceinline__ void nat_merge(const NatLookup &x, uint32_t out[4]) {
  out[0] = perm(x.hiA, x.loA, 0x05010400u);
  out[1] = perm(x.hiA, x.loA, 0x07030602u);
  out[2] = perm(x.hiB, x.loB, 0x05010400u);
  out[3] = perm(x.hiB, x.loB, 0x07030602u);
}

// Dequantize the 8 elements of one packed word w; out[j] = elem 2j |
// elem 2j+1 << 16, i.e. natural element order in memory.
__device__ __forceinline__ void lut_apply8(const Lut16 &t, uint32_t w, uint32_t out[4]) {
  WordLookup x;
  word_select(w, x);
  word_even(t, x);
  word_odd(t, x);
  word_merge(x, out);
}

// The product table built in 8 halves of quarters, for callers that
// interleave it with other work: half h computes entries 2h and 2h+1 into
// d[h & 1]; the odd half of quarter q then also forms lo[q] and hi[q].
template <bool kF16>
__device__ __forceinline__ void make_lut_half(float absmax, int h, uint32_t (&d)[2], Lut16 &t) {
  const float p0 = fp32_rounded(code_value(2 * h) * absmax);
  const float p1 = fp32_rounded(code_value(2 * h + 1) * absmax);
  d[h & 1] = kF16 ? pack_f16x2(p0, p1) : pack_bf16x2(p0, p1);
  if (h & 1) {
    t.lo[h >> 1] = perm(d[1], d[0], 0x06040200u);
    t.hi[h >> 1] = perm(d[1], d[0], 0x07050301u);
  }
}

// The product table built in 4 quarters (entries 4q..4q+3 each), for callers
// that interleave it with other work.
template <bool kF16>
__device__ __forceinline__ void make_lut_quarter(float absmax, int q, Lut16 &t) {
  const float p0 = fp32_rounded(code_value(4 * q) * absmax);
  const float p1 = fp32_rounded(code_value(4 * q + 1) * absmax);
  const float p2 = fp32_rounded(code_value(4 * q + 2) * absmax);
  const float p3 = fp32_rounded(code_value(4 * q + 3) * absmax);
  const uint32_t d0 = kF16 ? pack_f16x2(p0, p1) : pack_bf16x2(p0, p1);
  const uint32_t d1 = kF16 ? pack_f16x2(p2, p3) : pack_bf16x2(p2, p3);
  t.lo[q] = perm(d1, d0, 0x06040200u);
  t.hi[q] = perm(d1, d0, 0x07050301u);
}

// Per-block absmax, fp32 or double-quantized: (float)q * scale[b >> shift]
// (groups of 2^shift blocks).
struct AbsmaxRef {
  const float *absmax;
  const uint8_t *q;
  const float *scale;
  int32_t group_shift;
  int32_t block_shift;  // fused GEMMs: log2(block_size / 64) (a block spans 2^shift steps)
};

__device__ __forceinline__ float load_absmax(const AbsmaxRef &a, int64_t blk) {
  if (a.q == nullptr) return a.absmax[blk];
  return (float)a.q[blk] * a.scale[blk >> a.group_shift];
}

}  // namespace nf4s
