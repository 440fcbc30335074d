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
 *     its inputs and writes only its outputs;
 *   - a call over zero elements or zero tokens reads no input and returns
 *     NF4S_OK; its empty buffers may then be NULL or unaligned (the weight
 *     gradient over zero tokens still sets dW to 0, or leaves it when
 *     accumulating).
 *
 * Paths in citations are relative to the AethelStream source tree.
 */
#ifndef NF4STREAM_H
#define NF4STREAM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NF4S_ABI_VERSION 3

enum nf4s_status {
    NF4S_OK = 0,
    NF4S_ERR_INVALID_ARGUMENT = 1,   /* null pointer, negative size, bad block size */
    NF4S_ERR_ABSMAX_TOO_SMALL = 2,   /* nf4.rs:46-51 MalformedIndex("nf4_absmax", ..) */
    NF4S_ERR_PACKED_TOO_SMALL = 3,   /* nf4.rs:52-57 MalformedIndex("nf4_packed", ..) */
    NF4S_ERR_MISALIGNED = 4,         /* pointer alignment a kernel requires */
    NF4S_ERR_UNSUPPORTED_SHAPE = 5,  /* shape outside what a kernel supports */
    NF4S_ERR_HIP = 6,                /* HIP runtime or launch error */
    NF4S_ERR_IO = 7,                 /* error.rs:7-9   ShardEngineError::Io */
    NF4S_ERR_JSON = 8,               /* error.rs:11-13 ShardEngineError::Json */
    NF4S_ERR_LAYER_NOT_FOUND = 9,    /* error.rs:15-17 ShardEngineError::LayerNotFound */
    NF4S_ERR_PARAM_NOT_FOUND = 10,   /* error.rs:19-21 ShardEngineError::ParamNotFound */
    NF4S_ERR_MALFORMED_INDEX = 11,   /* error.rs:23-25 MalformedIndex (index entries) */
    NF4S_ERR_PREFETCH_MISS = 12      /* flowcast/src/error.rs:20-25 FlowCastError::PrefetchMiss */
};

/* flowcast/src/config.rs:16-27 Precision, plus the NF4 of this path. */
enum nf4s_precision {
    NF4S_PRECISION_FP32 = 0,
    NF4S_PRECISION_FP16 = 1,
    NF4S_PRECISION_BF16 = 2,
    NF4S_PRECISION_INT8 = 3,
    NF4S_PRECISION_INT4 = 4,
    NF4S_PRECISION_NF4 = 5
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

/* Message of the last call made on this host thread: the reason it failed
 * (the reference's MalformedIndex detail text, e.g. "absmax too small:
 * 3 < 4"), or "" when it succeeded.  Every status-returning call clears it
 * first. */
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
 * nf4s_quantize for bfloat16 input (each value widened exactly to fp32 first),
 * block_size 64.  The weights a bf16 update leaves
 * (doublepass/src/precision.rs:187-202) re-quantize without an fp32 copy.
 */
int32_t nf4s_quantize_bf16(const uint16_t *x, int64_t n, int32_t block_size,
                           uint8_t *packed, float *absmax, void *stream);

/*
 * Quantize + double-quant in one launch (block_size 64, group a power of two
 * <= 8192): packed codes, uint8 absmax codes and one fp32 scale per group,
 * bit-identical to nf4s_quantize followed by nf4s_dq_encode, written into the
 * caller's buffers without scratch memory.  For weights modified by the
 * update step (doublepass/src/precision.rs:187-202) before their write-back
 * (FlowCast::on_weights_updated, flowcast/src/lib.rs:501-521).
 */
int32_t nf4s_quantize_dq(const float *x, int64_t n, int32_t block_size,
                         int32_t group, uint8_t *packed, uint8_t *absmax_q,
                         float *absmax_scale, void *stream);
int32_t nf4s_quantize_dq_bf16(const uint16_t *x, int64_t n, int32_t block_size,
                              int32_t group, uint8_t *packed,
                              uint8_t *absmax_q, float *absmax_scale,
                              void *stream);

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
 * Requires k % 64 == 0, block_size 64 << s (64 as the reference writes,
 * or 128, 256, ...; shard_engine/src/index.rs:33 lets the index name any)
 * with k % block_size == 0, x/y 16-byte aligned.  Block sizes above 64 run
 * the per-step weight loads (64 takes the batched ones).  Every GEMM
 * entry point takes m, n and k up to 2^39 (tile counts are 32-bit; the launch
 * also bounds the total of output tiles by 2^31 - 1) and rejects larger ones
 * with NF4S_ERR_UNSUPPORTED_SHAPE.
 */
int32_t nf4s_gemm_fwd(const uint16_t *x, const nf4s_tensor *w, int64_t m,
                      int64_t n, int64_t k, uint16_t *y, void *stream);

/*
 * Fused NF4 GEMM, input gradient: dx[m,k] (bf16) = dy[m,n] (bf16) . W,
 * W the NF4 tensor of shape [n,k], fp32 accumulation.
 * Replaces the dY.W loops of single_layer_backward
 * (doublepass/src/backward.rs:79-85,117-129,160-168,284-300).
 * Requires n % 64 == 0, k % 64 == 0, block_size 64 << s with
 * k % block_size == 0 (as nf4s_gemm_fwd).
 */
int32_t nf4s_gemm_dgrad(const uint16_t *dy, const nf4s_tensor *w, int64_t m,
                        int64_t n, int64_t k, uint16_t *dx, void *stream);

/*
 * Grouped forward: y_i[m, ns[i]] = x[m,k] . W_i^T for `count` (1..4) NF4
 * weights W_i [ns[i], k] that share the activation x, in one launch whose
 * output tiles span all the weights.  Replaces the matmul_tb calls that share
 * their input in single_layer_forward: q/k/v (doublepass/src/forward.rs:174-176)
 * and gate/up (forward.rs:251-252).  Same requirements as nf4s_gemm_fwd for
 * each weight; weights of different kinds (double-quantized or not) run as
 * one launch per kind.
 */
int32_t nf4s_gemm_fwd_grouped(const uint16_t *x, const nf4s_tensor *ws,
                              const int64_t *ns, uint16_t *const *ys,
                              int32_t count, int64_t m, int64_t k,
                              void *stream);

/*
 * Forward with SwiGLU fused into the epilogue: hidden[m, ff] (bf16) =
 * silu(x . Wg^T) * (x . Wu^T), the gate and up products in fp32 and never
 * written out.  Replaces the gate/up matmul_tb calls and the elementwise
 * silu * up of single_layer_forward (doublepass/src/forward.rs:251-254;
 * silu_f at doublepass/src/math.rs:91-93).  Wg and Wu are [ff, k], both
 * double-quantized or both not; requirements as nf4s_gemm_fwd.
 */
int32_t nf4s_gemm_fwd_swiglu(const uint16_t *x, const nf4s_tensor *w_gate,
                             const nf4s_tensor *w_up, int64_t m, int64_t ff,
                             int64_t k, uint16_t *hidden, void *stream);

/*
 * Summed input gradient: dx[m,k] = sum_i dy_i[m, ns[i]] . W_i for `count`
 * (1..4) NF4 weights W_i [ns[i], k], one launch, one fp32 accumulator per
 * output element, one bf16 rounding.  Replaces the accumulating dY.W loops
 * of single_layer_backward: d_h1 = dq.Wq + dk.Wk + dv.Wv
 * (doublepass/src/backward.rs:284-300) and d_h2 = d_gate.Wg + d_up.Wu
 * (backward.rs:117-129).  Each ns[i] % 64 == 0; the weights are all
 * double-quantized or all not.
 */
int32_t nf4s_gemm_dgrad_sum(const uint16_t *const *dys, const nf4s_tensor *ws,
                            const int64_t *ns, int32_t count, int64_t m,
                            int64_t k, uint16_t *dx, void *stream);

/*
 * nf4s_gemm_dgrad_sum with a workspace for a split-K last round.  When the
 * output tiles (512 rows x 128 columns of dx) leave a last round of r tiles
 * on fewer than half the compute units (few tokens: 256 tokens of a 70B
 * layer give 64 tiles), each of those tiles runs as S = CUs / r slices of
 * the weights' concatenated reduction (W_0's rows, then W_1's, ...), whose
 * fp32 partial tiles go to `workspace` and are summed (in slice order) by a
 * second kernel on the same stream.  No counterpart in the reference: it
 * only reorders the fp32 sums of backward.rs:79-85, 117-129, 160-168 and
 * 284-300.  workspace may be NULL or smaller than
 * nf4s_gemm_dgrad_workspace_size reports: the call then runs without the
 * split.  Calls that share a workspace must not overlap (one stream, or
 * ordered streams).
 */
int32_t nf4s_gemm_dgrad_sum_ws(const uint16_t *const *dys, const nf4s_tensor *ws,
                               const int64_t *ns, int32_t count, int64_t m,
                               int64_t k, uint16_t *dx, void *workspace,
                               int64_t workspace_bytes, void *stream);

/*
 * Workspace bytes nf4s_gemm_dgrad_sum_ws uses for these shapes (0: no
 * split).  No device access.
 */
int32_t nf4s_gemm_dgrad_workspace_size(const int64_t *ns, int32_t count,
                                       int64_t m, int64_t k, int64_t *bytes);

/*
 * nf4s_gemm_fwd_grouped with a workspace for a split-K last round.  When the
 * output tiles leave a last round of r tiles on fewer than half the compute
 * units, each of those tiles runs as S = CUs / r slices of its reduction,
 * whose fp32 partial tiles go to `workspace` and are summed (in slice order)
 * by a second kernel on the same stream.  No counterpart in the reference:
 * it only reorders matmul_tb's fp32 sum (doublepass/src/math.rs:9-21).
 * workspace may be NULL or smaller than nf4s_gemm_fwd_workspace_size
 * reports: the call then runs without the split.  Calls that share a
 * workspace must not overlap (one stream, or ordered streams).
 */
int32_t nf4s_gemm_fwd_grouped_ws(const uint16_t *x, const nf4s_tensor *ws,
                                 const int64_t *ns, uint16_t *const *ys,
                                 int32_t count, int64_t m, int64_t k,
                                 void *workspace, int64_t workspace_bytes,
                                 void *stream);
/* Workspace bytes nf4s_gemm_fwd_grouped_ws uses for these shapes on the
 * current device (0: no split would help).  Allocates nothing. */
int32_t nf4s_gemm_fwd_workspace_size(const int64_t *ns, int32_t count, int64_t m,
                                     int64_t k, int64_t *bytes);

/*
 * nf4s_gemm_fwd_grouped_ws whose split-K workspace is the library's own
 * static device array (64 MiB per GPU) instead of a caller buffer: this call
 * allocates nothing, ever.  The array is reserved on a GPU by the first call
 * of this entry point there (with the code object that holds it) and held
 * until the process ends; a process that never calls it holds none of it.
 * No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Fails with
 * NF4S_ERR_UNSUPPORTED_SHAPE when the split needs more than the array holds
 * (possible only on devices with more than 256 CUs).  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (different streams
 * without ordering, or several host threads) race.  Results are bit-identical
 * to nf4s_gemm_fwd_grouped_ws with a large enough workspace.  The array's
 * device address is looked up on every call (valid across hipDeviceReset).
 * Under HIP graph capture: make one call of this entry point on the device
 * before capturing, so that the code objects of the array and of the GEMM
 * kernels are already loaded there; the call itself issues only kernel
 * launches (no memset), so a captured call replays correctly.
 */
int32_t nf4s_gemm_fwd_grouped_noalloc(const uint16_t *x, const nf4s_tensor *ws,
                                      const int64_t *ns, uint16_t *const *ys,
                                      int32_t count, int64_t m, int64_t k,
                                      void *stream);

/*
 * Weight gradient, bf16 in, fp32 out: dw[n, k] = sum_m dy[m, n] * x[m, k]
 * (accumulate = 0), or dw += that sum (accumulate != 0).  Replaces the d_wd,
 * d_wg / d_wu, d_wo and d_wq / d_wk / d_wv loops of single_layer_backward
 * (doublepass/src/backward.rs:87-93, 117-129, 160-168, 284-300); accumulate
 * is the micro-batch sum of backward.rs:478-502.  dy [m, n] and x [m, k] are
 * row-major bf16 with n % 8 == 0 and k % 8 == 0, 16-byte aligned; dw [n, k]
 * row-major fp32.  dy and x must each be below 2 GiB with m rounded up to a
 * multiple of 32.  No NF4 operand: this is the plain bf16 GEMM the backward
 * pass needs beside the fused ones.
 */
int32_t nf4s_gemm_wgrad(const void *dy, const void *x, int64_t m, int64_t n,
                        int64_t k, float *dw, int32_t accumulate, void *stream);

/*
 * Weight gradients of up to 4 products that share x, in one launch:
 * dws[i][ns[i], k] (+)= dys[i]^T . x, each as nf4s_gemm_wgrad computes it
 * (bit-identical).  Replaces the d_wq / d_wk / d_wv loops of
 * single_layer_backward, which all read the attention input
 * (doublepass/src/backward.rs:284-300), and d_wg / d_wu, which read the MLP
 * input (:117-129).  The products' dW tiles share the launch's rounds, so
 * the narrow k and v products (1024 rows on 70B) do not each leave half the
 * GPU idle.  Requirements per product as nf4s_gemm_wgrad; count in [1, 4].
 */
int32_t nf4s_gemm_wgrad_grouped(const void *const *dys, const int64_t *ns,
                                float *const *dws, int32_t count, const void *x,
                                int64_t m, int64_t k, int32_t accumulate,
                                void *stream);

/*
 * RMSNorm forward producing the fused GEMMs' bf16 operand: for each row b of
 * x [m, d] (fp32), rms[b] = sqrt(sum_i x[b,i]^2 / d + eps) and y[b,i] =
 * bf16((x[b,i] / rms[b]) * w[i]), fp32 arithmetic with correctly rounded
 * division and square root.  Replaces rms_norm_fwd
 * (doublepass/src/math.rs:28-59) at forward.rs:173 and :249, whose outputs
 * feed the q/k/v and gate/up GEMMs; rms (fp32, m values) is kept for the
 * backward.  The squares are summed as a tree, not in index order.
 * Requires d % 4 == 0, d <= 32768, x and w 16-byte aligned, y 8-byte aligned.
 */
int32_t nf4s_rmsnorm_fwd(const float *x, const float *w, int64_t m, int64_t d, float eps,
                         uint16_t *y, float *rms, void *stream);

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
 * when len exceeds the slot capacity (vram_double_buffer.rs:269-275), and
 * when the staging slot was handed out and not released yet.  The slot
 * returned at call N is refilled at call N+2, after the copy stream has
 * waited for the release recorded for it.
 */
int32_t nf4s_dbuf_advance(nf4s_dbuf *d, uint32_t layer_idx, const void *src,
                          int64_t len, void **dev_ptr, void **ready_event);

/* Records that everything enqueued so far on `compute_stream` is the last use
 * of the slot at `dev_ptr` (returned by nf4s_dbuf_advance); the copy that
 * refills that slot waits for this.  Once per advance. */
int32_t nf4s_dbuf_release(nf4s_dbuf *d, const void *dev_ptr, void *compute_stream);

/* FlowCast's ReadyLayer (flowcast/src/ready.rs:20-52) with the
 * cuda-double-buffer feature: slab 0 is the double-buffer slot holding the
 * layer's blob, and the consumer must make its compute stream wait on
 * `copy_event` before reading it (ready.rs:16-19). */
typedef struct nf4s_ready_layer {
    uint32_t layer_idx;
    void *slab_device_ptr;   /* slab 0 (ready.rs:32-36) */
    int64_t bytes;           /* blob bytes copied into the slot */
    void *copy_event;        /* hipEvent_t (ready.rs:43-51) */
    int32_t precision;       /* an nf4s_precision value; ready.rs:25-26 */
    int32_t needs_decode;    /* 1 for INT4 / INT8 (ready.rs:38-41, decode.rs:181-183) */
} nf4s_ready_layer;

/* FlowCast::take_ready (flowcast/src/lib.rs:458-498) over the double buffer,
 * for a blob the caller holds resident: nf4s_dbuf_advance of the layer's
 * pinned blob, returned as a ReadyLayer of precision NF4 (needs_decode 0:
 * the fused GEMMs dequantize in-kernel).  Fails like nf4s_dbuf_advance
 * (capacity; a staging slot whose previous layer was not retired). */
int32_t nf4s_take_ready(nf4s_dbuf *d, uint32_t layer_idx, const void *pinned,
                        int64_t len, nf4s_ready_layer *out);

/*
 * Residency table: the layers whose blobs a prefetcher has made resident in
 * pinned host memory, the ready map of FlowCast's prefetch state machine
 * (flowcast/src/state_machine.rs:306-346 is_ready / take_slot).  Host-only
 * and thread-safe: one thread may publish while another waits.  Destroy it
 * only when no other thread uses it.
 */
typedef struct nf4s_residency nf4s_residency;
int32_t nf4s_residency_create(uint32_t num_layers, nf4s_residency **out);
int32_t nf4s_residency_destroy(nf4s_residency *r);
/* Marks layer `layer_idx` resident: its blob is `bytes` at `pinned`, decoded
 * in `precision`.  Wakes a waiter.  Fails for an index beyond the table or a
 * layer already resident (not yet taken). */
int32_t nf4s_residency_publish(nf4s_residency *r, uint32_t layer_idx,
                               const void *pinned, int64_t bytes,
                               int32_t precision);
/* The state machine's take_ready (state_machine.rs:306-346): waits until the
 * layer is resident, then takes it (a second wait for it waits for the next
 * publish).  As the reference, the deadline is checked before readiness, so
 * timeout_us = 0 always misses; past the deadline it returns
 * NF4S_ERR_PREFETCH_MISS with the message "prefetch miss on layer N".
 * Timeouts above 10^15 us (about 31 years) wait that long. */
int32_t nf4s_residency_wait(nf4s_residency *r, uint32_t layer_idx,
                            int64_t timeout_us, const void **pinned,
                            int64_t *bytes, int32_t *precision);

/* FlowCast::take_ready (flowcast/src/lib.rs:458-498) in full:
 * nf4s_residency_wait, then nf4s_dbuf_advance of the taken blob.  The
 * ReadyLayer carries the published precision and needs_decode =
 * (precision is INT4 or INT8), as QuantizedDecoder::needs_decode.  A layer
 * whose copy then fails (capacity, unreleased slot) stays taken, as the
 * reference drops the taken slot when its advance fails. */
int32_t nf4s_take_ready_wait(nf4s_dbuf *d, nf4s_residency *r, uint32_t layer_idx,
                             int64_t timeout_us, nf4s_ready_layer *out);

/* FlowCast::retire_layer (flowcast/src/lib.rs:543-545): the work enqueued so
 * far on `compute_stream` is the layer's last use (nf4s_dbuf_release of its
 * slot).  Fails for a layer already retired or whose slot was refilled. */
int32_t nf4s_retire_layer(nf4s_dbuf *d, const nf4s_ready_layer *layer,
                          void *compute_stream);

/* hipStreamWaitEvent on a ready event returned by nf4s_dbuf_advance. */
int32_t nf4s_stream_wait_event(void *stream, void *event);

/* ---------------------------------------------------------------------------
 * Shard loader: the reference's on-disk NF4 format (shard_index.json +
 * layer_registry.json + safetensors shards; shard_engine/src/index.rs:7-34,
 * shard_engine/python/pipeline/writer.py:29-48,72-132), files mmap'd, NF4
 * dequantized on the device.  A loader is used from one stream at a time
 * (the reference's ShardLoader takes &mut self, loader.rs:36-40).
 * ------------------------------------------------------------------------- */
typedef struct nf4s_loader nf4s_loader;

typedef struct nf4s_param_info {
    int64_t shape[8];
    int32_t ndim;
    int32_t precision;     /* 0 fp16, 1 nf4, 2 nf4 with double-quant absmax */
    int64_t numel;
    int64_t byte_length;   /* TensorInfo.byte_length (packed bytes for nf4) */
    int64_t absmax_len;    /* fp32 absmax entries, or double-quant codes */
    int64_t scale_len;     /* double-quant fp32 scales */
    int32_t block_size;
    int32_t dq_group;
    int64_t out_elems;     /* f16 elements load_param yields (2 * packed bytes for nf4) */
    char precision_str[16];/* TensorInfo.precision ("nf4", "fp16", ...), NUL-terminated */
    char dtype_str[16];    /* TensorInfo.dtype */
} nf4s_param_info;

/* ShardLoader::new (shard_engine/src/loader.rs:44-50): reads
 * shard_index.json and layer_registry.json (index.rs:279-295). */
int32_t nf4s_loader_open(const char *model_dir, nf4s_loader **out);
int32_t nf4s_loader_close(nf4s_loader *l);

/* IndexStore::tensor_info (index.rs:307-311) as a plain struct. */
int32_t nf4s_loader_param_info(nf4s_loader *l, const char *name, nf4s_param_info *out);

/* ShardLoader::load_layer (loader.rs:53-75): the layer's whole shard file
 * (safetensors bytes), as a read-only mapping valid until nf4s_loader_close. */
int32_t nf4s_loader_load_layer(nf4s_loader *l, uint32_t layer, const uint8_t **data,
                               int64_t *len);

/* Device staging bytes nf4s_loader_load_param_f16 needs for `name`: the
 * packed bytes, absmax part and scales at 256-byte boundaries (0 for an fp16
 * entry).  An NF4 entry is first checked against its shard file, with the
 * errors nf4s_loader_load_param_f16 reports.  Allocates nothing. */
int32_t nf4s_loader_staging_size(nf4s_loader *l, const char *name, int64_t *bytes);

/* ShardLoader::load_param (loader.rs:78-206) into a device f16 buffer of
 * out_len elements: NF4 entries pass the reference's checks in its order
 * (loader.rs:99-151), are copied into the caller's 16-byte aligned device
 * `staging` buffer (at least nf4s_loader_staging_size bytes) and dequantized
 * on the device with dequant_nf4_alloc semantics (2 * packed bytes elements,
 * nf4.rs:98-107); fp16 entries are copied (loader.rs:179-198).  Calls that
 * share a staging buffer must not overlap (one stream, or ordered streams). */
int32_t nf4s_loader_load_param_f16(nf4s_loader *l, const char *name, uint16_t *out,
                                   int64_t out_len, void *staging, int64_t staging_bytes,
                                   void *stream);

/* The raw NF4 payload of a parameter (packed bytes, fp32 absmax or uint8
 * codes, fp32 scales) copied into caller device buffers of the given byte
 * capacities, for a weight provider that keeps NF4 resident instead of
 * widening it to f32 (doublepass/src/shard_provider.rs:103-130).  The fp32
 * parts copy floor(length / 4) floats, what the reference reads
 * (loader.rs:158-161); `scale` is NULL (capacity 0) without double-quant. */
int32_t nf4s_loader_load_param_nf4(nf4s_loader *l, const char *name, uint8_t *packed,
                                   int64_t packed_bytes, void *absmax_or_q,
                                   int64_t absmax_bytes, float *scale, int64_t scale_bytes,
                                   void *stream);

/* Placement of one NF4 parameter in a layer blob, byte offsets from the
 * blob start; each part begins at a 256-byte boundary. */
typedef struct nf4s_blob_entry {
    int64_t packed_off;
    int64_t packed_len;    /* bytes */
    int64_t absmax_off;    /* fp32 absmax, or uint8 double-quant codes */
    int64_t absmax_len;    /* entries */
    int64_t scale_off;     /* fp32 double-quant scales (0 without) */
    int64_t scale_len;     /* entries (0 without double-quant) */
    int32_t block_size;
    int32_t dq_group;      /* 0 without double-quant */
} nf4s_blob_entry;

/* The bytes a FlowCast pinned slot holds for one layer
 * (flowcast/src/ready.rs:27-30): the raw NF4 payloads of `count` parameters
 * (e.g. a layer's 7 matrices) copied from the mmap'd shards into one host
 * blob `dst` (pinned, so that nf4s_take_ready copies it asynchronously),
 * parts placed as nf4s_blob_entry says.  With dst == NULL only `entries` and
 * *bytes are filled (a size query).  Entries pass the checks of
 * nf4s_loader_load_param_nf4. */
int32_t nf4s_loader_pack_layer(nf4s_loader *l, const char *const *names, int32_t count,
                               void *dst, int64_t dst_bytes, nf4s_blob_entry *entries,
                               int64_t *bytes);

/* Descriptor of blob entry `e` inside a copy of the blob at `base` (e.g. the
 * slab of a ReadyLayer). */
int32_t nf4s_blob_tensor(const nf4s_blob_entry *e, const void *base, nf4s_tensor *out);

#ifdef __cplusplus
}
#endif
#endif
