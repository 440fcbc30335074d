// nf4_noalloc.hip - nf4s_gemm_fwd_grouped_noalloc: the grouped split-K forward
// GEMM (nf4_gemm.hip) with the library's own static device array as its
// workspace, for callers that cannot allocate.  No counterpart in the
// reference.
//
// The array is the only device object of this file, so it sits in a code
// object of its own.  HIP loads a code object on a GPU, and reserves its
// device memory there, the first time the object is used on that GPU: here,
// the first lookup of the array.  A process that never calls this entry
// point holds none of the 64 MiB; one that does holds it on each GPU it
// called it on until the process ends.
#include "abi_common.hpp"

namespace nf4s {

// A split plan never needs more partial tiles than the device has CUs
// (S <= CUs / r slices for r tail tiles), so 256 partial tiles (64 MiB)
// cover every shape on a 256-CU MI355X.
constexpr int64_t kScratchTiles = 256;
constexpr int64_t kScratchBytes = kScratchTiles * kGemmPartialTileBytes;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

// Device address of the current GPU's `scratch`, looked up on every call
// with that device current: each GPU holds its own copy at its own address,
// and a hipDeviceReset reloads the code object (a cached address would then
// dangle).  The lookup is a host-side table query once the code object is
// loaded, small next to a GEMM launch.  The host-side name is only a
// stand-in handle: kernels get this address, never the name.
static int32_t scratch_on_current_device(void **out) {
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr)
    return fail(NF4S_ERR_HIP, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
  *out = p;
  return NF4S_OK;
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

// nf4s_gemm_fwd_grouped_ws with the static per-GPU scratch as the workspace.
// Sizes beyond the scratch are rejected before the array is looked up, so a
// rejected call loads nothing.
int32_t nf4s_gemm_fwd_grouped_noalloc(const uint16_t *x, const nf4s_tensor *ws, const int64_t *ns,
                                      uint16_t *const *ys, int32_t count, int64_t m, int64_t k,
                                      void *stream) {
  clear_error();
  int64_t need = 0;
  int32_t rc = fwd_workspace_query(ns, count, m, k, &need);
  if (rc != NF4S_OK) return rc;
  if (need > kScratchBytes)
    return fail(NF4S_ERR_UNSUPPORTED_SHAPE,
                "split-K workspace of %lld bytes exceeds the static scratch of %lld bytes; "
                "use nf4s_gemm_fwd_grouped_ws with a workspace of that size",
                (long long)need, (long long)kScratchBytes);
  void *p = nullptr;
  rc = scratch_on_current_device(&p);
  if (rc != NF4S_OK) return rc;
  return gemm_fwd_grouped_on(x, ws, ns, ys, count, m, k, as_stream(stream), p, kScratchBytes);
}

}  // extern "C"
