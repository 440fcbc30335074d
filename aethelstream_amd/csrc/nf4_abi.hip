// nf4_abi.hip - version, status strings and argument validation of the C ABI.
#include "abi_common.hpp"

namespace nf4s {

static thread_local char g_msg[512] = "";

int32_t fail(int32_t rc, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return rc;
}

void clear_error() { g_msg[0] = '\0'; }

int32_t check_launch(const char *what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(NF4S_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return NF4S_OK;
}

int32_t validate_tensor(const nf4s_tensor *t, int64_t n) {
  if (t == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "tensor descriptor is NULL");
  if (n < 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "negative element count %lld", (long long)n);
  if (t->block_size <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "block_size must be positive, got %d", t->block_size);
  if (t->packed_len < 0 || t->absmax_len < 0 || t->scale_len < 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "negative buffer length");
  const bool dq = t->absmax_q != nullptr;
  // An empty tensor's buffers may all be NULL (an empty tensor's data
  // pointer is), so the rule only binds when there are elements.
  if (n > 0 && dq == (t->absmax != nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "exactly one of absmax / absmax_q must be set");
  // shard_engine/src/nf4.rs:43-57, same order and wording.
  const int64_t nb = ceil_div(n, t->block_size);
  if (t->absmax_len < nb)
    return fail(NF4S_ERR_ABSMAX_TOO_SMALL, "absmax too small: %lld < %lld",
                (long long)t->absmax_len, (long long)nb);
  if (t->packed_len < ceil_div(n, 2))
    return fail(NF4S_ERR_PACKED_TOO_SMALL, "packed too small: %lld < %lld",
                (long long)(t->packed_len * 2), (long long)n);
  if (n > 0 && t->packed == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "packed is NULL");
  if (dq) {
    if (t->dq_group <= 0 || (t->dq_group & (t->dq_group - 1)) != 0)
      return fail(NF4S_ERR_INVALID_ARGUMENT, "dq_group must be a power of two, got %d",
                  t->dq_group);
    const int64_t ng = ceil_div(nb, t->dq_group);
    if (t->scale_len < ng || (ng > 0 && t->absmax_scale == nullptr))
      return fail(NF4S_ERR_ABSMAX_TOO_SMALL, "absmax scale too small: %lld < %lld",
                  (long long)t->scale_len, (long long)ng);
  }
  return NF4S_OK;
}

}  // namespace nf4s

extern "C" {

int32_t nf4s_abi_version(void) { return NF4S_ABI_VERSION; }

const char *nf4s_strerror(int32_t status) {
  switch (status) {
    case NF4S_OK: return "ok";
    case NF4S_ERR_INVALID_ARGUMENT: return "invalid argument";
    case NF4S_ERR_ABSMAX_TOO_SMALL: return "malformed index: nf4_absmax";
    case NF4S_ERR_PACKED_TOO_SMALL: return "malformed index: nf4_packed";
    case NF4S_ERR_MISALIGNED: return "misaligned pointer";
    case NF4S_ERR_UNSUPPORTED_SHAPE: return "unsupported shape";
    case NF4S_ERR_HIP: return "HIP runtime error";
    case NF4S_ERR_IO: return "I/O error";
    case NF4S_ERR_JSON: return "JSON parse error";
    case NF4S_ERR_LAYER_NOT_FOUND: return "layer index not found in layer registry";
    case NF4S_ERR_PARAM_NOT_FOUND: return "parameter not found in shard index";
    case NF4S_ERR_MALFORMED_INDEX: return "malformed index entry";
    case NF4S_ERR_PREFETCH_MISS: return "prefetch miss";
    default: return "unknown status";
  }
}

const char *nf4s_last_error_message(void) { return nf4s::g_msg; }

}  // extern "C"
