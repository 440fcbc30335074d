// abi_common.hpp - host-side helpers shared by the extern "C" entry points:
// status codes, the per-thread error message, and nf4s_tensor validation
// mirroring shard_engine/src/nf4.rs:43-57.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/nf4stream.h"

namespace nf4s {

// Formats the message returned by nf4s_last_error_message() and returns rc.
int32_t fail(int32_t rc, const char *fmt, ...);

// Empties the message of nf4s_last_error_message(); every status-returning
// entry point calls it first, so the message always belongs to the last call
// made on this thread and is empty after a successful one.
void clear_error();

inline hipStream_t as_stream(void *s) { return reinterpret_cast<hipStream_t>(s); }

// Launch status of the kernel just enqueued.
int32_t check_launch(const char *what);

inline bool aligned(const void *p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ceil(a / b) for a >= 0, b > 0, without the a + b - 1 that wraps for
// caller sizes near 2^63.
inline int64_t ceil_div(int64_t a, int64_t b) { return a / b + (a % b != 0 ? 1 : 0); }

// log2 of a power-of-two double-quant group (validate_tensor checks it).
inline int32_t group_shift(int32_t group) {
  int32_t s = 0;
  while ((1 << s) < group) ++s;
  return s;
}

// Validates `t` for reading n elements: the two MalformedIndex checks of
// shard_engine/src/nf4.rs:46-57 (same order, same message text), plus the
// pointer and double-quant fields.
int32_t validate_tensor(const nf4s_tensor *t, int64_t n);

// The grouped forward GEMM of nf4_gemm.hip, for the no-allocation entry point
// in nf4_noalloc.hip.  fwd_workspace_query checks count and ns and sets
// *bytes to the split-K workspace that nf4s_gemm_fwd_grouped_ws would use
// (nf4s_gemm_fwd_workspace_size); gemm_fwd_grouped_on runs that entry
// point's launches on the given workspace.
int32_t fwd_workspace_query(const int64_t *ns, int32_t count, int64_t m, int64_t k,
                            int64_t *bytes);
int32_t gemm_fwd_grouped_on(const uint16_t *x, const nf4s_tensor *ws, const int64_t *ns,
                            uint16_t *const *ys, int32_t count, int64_t m, int64_t k,
                            hipStream_t s, void *work, int64_t work_bytes);
// One split-K partial tile of the forward GEMM: 256 threads x 256 fp32
// accumulators (a 512 x 128 output tile).
constexpr int64_t kGemmPartialTileBytes = 256 * 256 * 4;

}  // namespace nf4s
