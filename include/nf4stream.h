/*
 * nf4stream.h - C ABI of the MI355X (gfx950) NF4 streamed-weight library
 * (libnf4stream.so).
 *
 * Conventions, following the reference's Rust->native FFI
 * (galore/src/kernels/mod.rs:6-50, ramflow/src/cuda_bridge/stream.rs:83):
 *   - every entry point returns int32_t status, 0 = NF4S_OK;
 *   - device buffers are plain pointers, sizes are int64_t element counts,
 *     the HIP stream is passed as void* (NULL = the default stream);
 *   - calls are stream-ordered and asynchronous unless stated otherwise;
 *     they allocate no device memory and let no C++ exception escape;
 *   - calls on different streams may run concurrently; each call reads only
 *     its inputs and writes only its outputs.
 *
 * Paths in citations are relative to the AethelStream source tree.
 */
#ifndef NF4STREAM_H
#define NF4STREAM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NF4S_ABI_VERSION 1

enum nf4s_status {
    NF4S_OK = 0,
    NF4S_ERR_INVALID_ARGUMENT = 1,   /* null pointer, negative size, bad block size */
    NF4S_ERR_ABSMAX_TOO_SMALL = 2,   /* nf4.rs:46-51 MalformedIndex("nf4_absmax", ..) */
    NF4S_ERR_PACKED_TOO_SMALL = 3,   /* nf4.rs:52-57 MalformedIndex("nf4_packed", ..) */
    NF4S_ERR_MISALIGNED = 4,         /* pointer alignment a kernel requires */
    NF4S_ERR_UNSUPPORTED_SHAPE = 5,  /* shape outside what a kernel supports */
    NF4S_ERR_HIP = 6                 /* HIP runtime or launch error */
};

/*
 * One NF4 tensor resident in device memory: the on-disk payload of
 * shard_engine/src/index.rs:7-34 (`{p}.__packed__` U8, `{p}.__absmax__` F32,
 * shard_engine/python/pipeline/writer.py:72-84), optionally with the absmax
 * double-quantized (uint8 codes 0..127 per block, one fp32 scale per
 * `dq_group` blocks).  Element e sits in byte e/2, high nibble for even e
 * (shard_engine/src/nf4.rs:66-74); block b covers elements [b*bs, (b+1)*bs).
 * Exactly one of `absmax` / `absmax_q` is non-NULL.
 */
typedef struct nf4s_tensor {
    const uint8_t *packed;      /* packed nibbles */
    int64_t packed_len;         /* bytes in `packed` */
    const float *absmax;        /* fp32 per block, or NULL */
    const uint8_t *absmax_q;    /* double-quant code per block, or NULL */
    const float *absmax_scale;  /* fp32 per dq_group blocks (with absmax_q) */
    int64_t absmax_len;         /* entries in absmax / absmax_q */
    int64_t scale_len;          /* entries in absmax_scale (0 without dq) */
    int32_t block_size;         /* elements per block (64 in the reference) */
    int32_t dq_group;           /* blocks per scale, a power of two (256); 0 without dq */
} nf4s_tensor;

/* NF4S_ABI_VERSION of the loaded library. */
int32_t nf4s_abi_version(void);

/* Static description of a status code. */
const char *nf4s_strerror(int32_t status);

/* Message of the last failing call on this host thread (the reference's
 * MalformedIndex detail text, e.g. "absmax too small: 3 < 4"). */
const char *nf4s_last_error_message(void);

/*
 * NF4 blockwise quantize on the device.
 * Replaces quantize_nf4 (shard_engine/python/pipeline/quantizer.py:21-53):
 * x (n fp32) -> packed (ceil(n/2) bytes, high nibble first, code-0 pad
 * nibble for odd n) and absmax (ceil(n/block_size) fp32, unclamped max |x|
 * of each zero-padded block).  Codes are the first-index argmin of
 * |x/max(absmax,1e-8) - code_i| in fp32, bit-exact with the reference.
 */
int32_t nf4s_quantize(const float *x, int64_t n, int32_t block_size,
                      uint8_t *packed, float *absmax, void *stream);

/*
 * Double-quantize per-block absmax: groups of `group` blocks, scale =
 * max/127 (1.0 for an all-zero group), q = clamp(rne(absmax/scale), 0, 127).
 * No counterpart in the reference (its index holds fp32 absmax only,
 * shard_engine/src/index.rs:27-33); conventions from
 * galore/src/quantize.rs:4-13.
 */
int32_t nf4s_dq_encode(const float *absmax, int64_t nblocks, int32_t group,
                       uint8_t *q, float *scale, void *stream);

/*
 * Dequantize n elements of `t` to IEEE binary16 (RNE).
 * Replaces dequant_nf4_into (shard_engine/src/nf4.rs:37-83): out[e] =
 * f16(code[nibble(e)] * absmax[e / block_size]), one fp32 multiply; fails
 * with NF4S_ERR_ABSMAX_TOO_SMALL / NF4S_ERR_PACKED_TOO_SMALL exactly where
 * the reference returns MalformedIndex.  With n = 2 * packed_len this is
 * dequant_nf4_alloc (nf4.rs:98-107).
 */
int32_t nf4s_dequant_f16(const nf4s_tensor *t, int64_t n, uint16_t *out,
                         void *stream);

/* Same as nf4s_dequant_f16 with bfloat16 (RNE) output: the GEMM operand. */
int32_t nf4s_dequant_bf16(const nf4s_tensor *t, int64_t n, uint16_t *out,
                          void *stream);

/*
 * Dequantize `count` tensors (e.g. the 7 matrices of one decoder layer) in one
 * launch, bf16 output.  Replaces the per-parameter load_param loop of
 * doublepass/src/shard_provider.rs:103-130 with one grouped kernel.
 */
int32_t nf4s_dequant_batch_bf16(const nf4s_tensor *ts, const int64_t *ns,
                                uint16_t *const *outs, int32_t count,
                                void *stream);

/*
 * Fused NF4 GEMM, forward: y[m,n] (bf16) = x[m,k] (bf16) . W^T, W the NF4
 * tensor `w` of shape [n,k] row-major, fp32 accumulation.
 * Replaces matmul_tb (doublepass/src/math.rs:9-21) at its call sites in
 * single_layer_forward (doublepass/src/forward.rs:174-176,244,251-252,255) and
 * the recompute forward (doublepass/src/backward.rs:447-451).
 * Requires k % 64 == 0, block_size == 64, x/y 16-byte aligned.
 */
int32_t nf4s_gemm_fwd(const uint16_t *x, const nf4s_tensor *w, int64_t m,
                      int64_t n, int64_t k, uint16_t *y, void *stream);

/*
 * Fused NF4 GEMM, input gradient: dx[m,k] (bf16) = dy[m,n] (bf16) . W,
 * W the NF4 tensor of shape [n,k], fp32 accumulation.
 * Replaces the dY.W loops of single_layer_backward
 * (doublepass/src/backward.rs:79-85,117-129,160-168,284-300).
 * Requires n % 64 == 0, k % 64 == 0, block_size == 64.
 */
int32_t nf4s_gemm_dgrad(const uint16_t *dy, const nf4s_tensor *w, int64_t m,
                        int64_t n, int64_t k, uint16_t *dx, void *stream);

/* ---------------------------------------------------------------------------
 * Streamed layer stack (one GPU).  Layers wait in pinned host memory and are
 * copied into a two-slot device double buffer on a dedicated copy stream.
 * ------------------------------------------------------------------------- */

/* Pinned (page-locked) host memory of `bytes`; replaces PinnedBuffer::alloc
 * (ramflow/src/allocator/pinned.rs:306) for the H2D source buffers. */
int32_t nf4s_host_alloc(int64_t bytes, void **out);
int32_t nf4s_host_free(void *p);

/* Two device slots of `slot_bytes`, a copy stream and per-slot events;
 * replaces VramDoubleBuffer::new (flowcast/src/vram_double_buffer.rs:230-237).
 * Allocates; the other dbuf calls do not. */
typedef struct nf4s_dbuf nf4s_dbuf;
int32_t nf4s_dbuf_create(int64_t slot_bytes, nf4s_dbuf **out);
int32_t nf4s_dbuf_destroy(nf4s_dbuf *d);
int64_t nf4s_dbuf_capacity(const nf4s_dbuf *d);

/*
 * VramDoubleBuffer::advance (flowcast/src/vram_double_buffer.rs:263-301):
 * copies `len` bytes of host `src` (pinned for an asynchronous copy) into the
 * staging slot on the copy stream, records the slot's ready event, swaps the
 * slots and returns the new compute slot and its event.  The consumer must
 * make its compute stream wait on `*ready_event` (nf4s_stream_wait_event)
 * before reading `*dev_ptr` (flowcast/src/ready.rs:16-19,43-51).  Fails
 * when len exceeds the slot capacity (vram_double_buffer.rs:269-275).  The
 * slot returned at call N is refilled at call N+2, after the copy stream has
 * waited for the release recorded for it.
 */
int32_t nf4s_dbuf_advance(nf4s_dbuf *d, uint32_t layer_idx, const void *src,
                          int64_t len, void **dev_ptr, void **ready_event);

/* Records that everything enqueued so far on `compute_stream` is the last use
 * of the slot at `dev_ptr` (returned by nf4s_dbuf_advance); the copy that
 * refills that slot waits for this. */
int32_t nf4s_dbuf_release(nf4s_dbuf *d, const void *dev_ptr, void *compute_stream);

/* hipStreamWaitEvent on a ready event returned by nf4s_dbuf_advance. */
int32_t nf4s_stream_wait_event(void *stream, void *event);

#ifdef __cplusplus
}
#endif
#endif
