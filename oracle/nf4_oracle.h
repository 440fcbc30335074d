/*
 * nf4_oracle.h - CPU restatement of the AethelStream NF4 streamed-weight path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * or the timed CPU baseline.  The product (libnf4stream.so) never links it.
 *
 * Every function names the reference file:line it restates.  Paths are
 * relative to the AethelStream source tree (aethelStream/).
 *
 * Pinning (what checks each function against something other than itself):
 *   or_codebook          literal bit table of shard_engine/src/nf4.rs:6-23,
 *                        KAT nf4.rs:113-116 (index 7 is 0.0)
 *   or_quantize_nf4      brute-force 16-way argmin vs the bracket rule,
 *                        exhaustively over every fp32 in [-1, 1]; a torch
 *                        op-by-op restatement on seeded vectors (fixtures);
 *                        special cases (zero block, +-absmax, sizes) from
 *                        shard_engine/tests/test_nf4_fidelity.py:14-43;
 *                        MSE bound test_nf4_fidelity.py:5-12
 *   or_dequant_*         KATs nf4.rs:118-143; f16/bf16 RNE cross-checked
 *                        against numpy/torch conversions of the same fp32
 *   or_dq_encode/decode  PARITY UNPINNED against the reference (the reference
 *                        has no double-quant); pinned by its own invariants
 *                        (q in [0,127], group max -> 127, |a'-a| <= s2/2)
 *   or_matmul_tb         closed form vs fp64 numpy on small shapes
 *   or_dgrad             closed form vs fp64 numpy on small shapes
 *   or_wgrad             closed form vs fp64 numpy on small shapes; exact on
 *                        small-integer data
 *   or_rmsnorm_fwd       closed form vs fp64 numpy; exact special cases (a
 *                        zero row gives rms = sqrt(eps) and y = 0; a row of
 *                        equal values v gives x_hat = v / sqrt(v^2 + eps))
 */
#ifndef NF4_ORACLE_H
#define NF4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* NF4 codebook, fp32, ascending (shard_engine/src/nf4.rs:6-23). */
void or_codebook(float out[16]);

/* IEEE-754 binary32 -> binary16 / bfloat16, round to nearest even. */
uint16_t or_f32_to_f16(float x);
uint16_t or_f32_to_bf16(float x);
float or_bf16_to_f32(uint16_t h);
float or_f16_to_f32(uint16_t h);

/* NF4 code of one normalised value: literal 16-way argmin with the first
 * index winning ties (quantizer.py:40-41). */
uint8_t or_nf4_code_argmin(float n);
/* Same result via the bracketing pair only (the rule the GPU kernel uses). */
uint8_t or_nf4_code_bracket(float n);

/* Exhaustive check of or_nf4_code_bracket against or_nf4_code_argmin over
 * every fp32 in [lo_bits..] of [-1, 1]; returns the number of mismatches.
 * nthreads <= 0 picks the OpenMP default. */
int64_t or_check_bracket_exhaustive(int nthreads);
int64_t or_check_steps_exhaustive(const float *steps, int nthreads);

/* quantize_nf4 (shard_engine/python/pipeline/quantizer.py:21-53).
 * x: n fp32 values.  packed: ceil(n/2) bytes.  absmax: ceil(n/bs) floats
 * (unclamped max |x| per zero-padded block). */
void or_quantize_nf4(const float *x, int64_t n, int32_t bs,
                     uint8_t *packed, float *absmax);

/* Double-quant encode of per-block absmax into uint8 codes (0..127) in
 * groups of `group` blocks, one fp32 scale per group.  Conventions from
 * galore/src/quantize.rs:4-13 (scale = max/127, 1.0 for an all-zero group)
 * with round-half-even as galore/kernels/quantize_state.cu:43. */
void or_dq_encode(const float *absmax, int64_t nblocks, int32_t group,
                  uint8_t *q, float *scale);
/* absmax' = (float)q * scale[block / group]. */
void or_dq_decode(const uint8_t *q, const float *scale, int64_t nblocks,
                  int32_t group, float *absmax_out);

/* dequant_nf4_into (shard_engine/src/nf4.rs:37-83) with the output
 * conversion chosen by the suffix: f16 is the reference (nf4.rs:78),
 * bf16 is the GEMM operand.  Returns 0, or 1 if absmax is too small, 2 if
 * packed is too small (the two MalformedIndex errors of nf4.rs:46-57). */
int or_dequant_f16(const uint8_t *packed, int64_t packed_len,
                   const float *absmax, int64_t absmax_len,
                   uint16_t *out, int64_t n, int32_t bs);
int or_dequant_bf16(const uint8_t *packed, int64_t packed_len,
                    const float *absmax, int64_t absmax_len,
                    uint16_t *out, int64_t n, int32_t bs);
/* fp32 product only (code * absmax), before any output conversion. */
int or_dequant_f32(const uint8_t *packed, int64_t packed_len,
                   const float *absmax, int64_t absmax_len,
                   float *out, int64_t n, int32_t bs);

/* matmul_tb (doublepass/src/math.rs:9-21): c[m,n] = a[m,k] . b[n,k]^T,
 * fp32, sequential sum over k. */
void or_matmul_tb(const float *a, const float *b, int64_t m, int64_t k,
                  int64_t n, float *c);

/* Input-gradient loop (doublepass/src/backward.rs:160-168):
 * dx[m,k] += dy[m,n] . w[n,k], fp32, for i, for j, for k order.
 * dx must be zeroed by the caller for a fresh result. */
void or_dgrad(const float *dy, const float *w, int64_t m, int64_t n,
              int64_t k, float *dx);

/* Weight-gradient loop (doublepass/src/backward.rs:87-93, d_wd):
 * dw[n,k] += dy[m,n] . x[m,k] summed over m, fp32, for n, for k, for m
 * order; the sites :117-129, :160-168 and :284-300 have the same form.
 * dw must be zeroed by the caller for a fresh result. */
void or_wgrad(const float *dy, const float *x, int64_t m, int64_t n,
              int64_t k, float *dw);

/* rms_norm_fwd (doublepass/src/math.rs:28-59): per row b of x [m, d],
 * mean_sq = (sum_i x^2) / d summed in index order, rms[b] = sqrt(mean_sq +
 * eps), x_hat = x / rms[b], y = x_hat * w[i]; fp32 throughout. */
void or_rmsnorm_fwd(const float *x, const float *w, int64_t m, int64_t d, float eps,
                    float *y, float *x_hat, float *rms);

/* Deterministic input generator: splitmix64(seed) -> 53-bit uniform ->
 * Box-Muller in fp64 -> * sigma -> fp32 round to nearest. */
void or_gen_normal(uint64_t seed, int64_t n, double sigma, float *out);

#ifdef __cplusplus
}
#endif
#endif
