// nf4_stream.hip - streamed layer stack on one GPU: pinned host layers, a
// two-slot device double buffer fed by a copy stream, events between the
// copy and compute streams.
//
// Mirrors flowcast's VramDoubleBuffer (flowcast/src/vram_double_buffer.rs:
// 196-301) with the real transfer the reference only declares
// (ramflow/src/cuda_bridge/bindings.rs:115-125,304-316):
//   advance(layer, src):  the copy stream waits until the staging slot is no
//   longer read by the compute stream, copies src into it (hipMemcpyAsync
//   H2D), records the slot's ready event, swaps the slots and returns the
//   new compute slot with its ready event.  The consumer makes its compute
//   stream wait on that event before reading the slot (ready.rs:16-19,43-51)
//   and calls release(slot) after enqueuing the kernels that read it.
// The buffer handed out at call N is overwritten at call N+2
// (vram_double_buffer.rs:258-262); release() turns that invariant into an
// event the copy stream waits on, so the host may run ahead of the GPU.
#include "abi_common.hpp"

#include <chrono>
#include <condition_variable>
#include <mutex>
#include <new>
#include <vector>

struct nf4s_dbuf {
  void *slot[2];          // device buffers
  hipEvent_t ready[2];    // copy into the slot complete
  hipEvent_t freed[2];    // last reader of the slot complete
  bool freed_valid[2];    // a release was recorded for the slot
  bool held[2];           // handed out by advance and not yet released
  uint32_t layer[2];      // layer index last copied into the slot
  int64_t capacity;
  int staging;            // index of slot_b (the next copy target)
  hipStream_t copy;
};

// The ready map of FlowCast's prefetch state machine
// (flowcast/src/state_machine.rs:306-346): per layer, the pinned blob a
// prefetcher published and its precision, until take_ready takes it.
struct nf4s_residency {
  struct Entry {
    bool resident = false;
    const void *pinned = nullptr;
    int64_t bytes = 0;
    int32_t precision = 0;
  };
  std::mutex mu;
  std::condition_variable cv;
  std::vector<Entry> layers;
};

namespace nf4s {

static int32_t hip_fail(hipError_t e, const char *what) {
  return fail(NF4S_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

}  // namespace nf4s

using namespace nf4s;

extern "C" {

int32_t nf4s_host_alloc(int64_t bytes, void **out) {
  clear_error();
  if (out == nullptr || bytes <= 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad host_alloc args");
  *out = nullptr;
  // Pinned (page-locked) host memory allocated as such; no hipHostRegister.
  const hipError_t e = hipHostMalloc(out, (size_t)bytes, hipHostMallocDefault);
  if (e != hipSuccess) return hip_fail(e, "hipHostMalloc");
  return NF4S_OK;
}

int32_t nf4s_host_free(void *p) {
  clear_error();
  if (p == nullptr) return NF4S_OK;
  const hipError_t e = hipHostFree(p);
  if (e != hipSuccess) return hip_fail(e, "hipHostFree");
  return NF4S_OK;
}

int32_t nf4s_dbuf_create(int64_t slot_bytes, nf4s_dbuf **out) {
  clear_error();
  if (out == nullptr || slot_bytes <= 0)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad dbuf_create args");
  *out = nullptr;
  nf4s_dbuf *d = new (std::nothrow) nf4s_dbuf();
  if (d == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "out of host memory");
  d->capacity = slot_bytes;
  d->staging = 1;
  hipError_t e = hipSuccess;
  for (int i = 0; i < 2 && e == hipSuccess; ++i) e = hipMalloc(&d->slot[i], (size_t)slot_bytes);
  for (int i = 0; i < 2 && e == hipSuccess; ++i)
    e = hipEventCreateWithFlags(&d->ready[i], hipEventDisableTiming);
  for (int i = 0; i < 2 && e == hipSuccess; ++i)
    e = hipEventCreateWithFlags(&d->freed[i], hipEventDisableTiming);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&d->copy, hipStreamNonBlocking);
  if (e != hipSuccess) {
    const int32_t rc = hip_fail(e, "dbuf_create");
    for (int i = 0; i < 2; ++i) {
      if (d->slot[i]) (void)hipFree(d->slot[i]);
      if (d->ready[i]) (void)hipEventDestroy(d->ready[i]);
      if (d->freed[i]) (void)hipEventDestroy(d->freed[i]);
    }
    delete d;
    return rc;
  }
  *out = d;
  return NF4S_OK;
}

int32_t nf4s_dbuf_destroy(nf4s_dbuf *d) {
  clear_error();
  if (d == nullptr) return NF4S_OK;
  hipError_t e = hipStreamSynchronize(d->copy);
  for (int i = 0; i < 2; ++i) {
    if (d->freed_valid[i]) (void)hipEventSynchronize(d->freed[i]);
    (void)hipFree(d->slot[i]);
    (void)hipEventDestroy(d->ready[i]);
    (void)hipEventDestroy(d->freed[i]);
  }
  (void)hipStreamDestroy(d->copy);
  delete d;
  if (e != hipSuccess) return hip_fail(e, "dbuf_destroy");
  return NF4S_OK;
}

int64_t nf4s_dbuf_capacity(const nf4s_dbuf *d) { return d ? d->capacity : 0; }

// vram_double_buffer.rs:263-301.
int32_t nf4s_dbuf_advance(nf4s_dbuf *d, uint32_t layer_idx, const void *src, int64_t len,
                          void **dev_ptr, void **ready_event) {
  clear_error();
  if (d == nullptr || dev_ptr == nullptr || ready_event == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad dbuf_advance args");
  if (len < 0 || (len > 0 && src == nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad source buffer");
  if (len > d->capacity)  // vram_double_buffer.rs:269-275, same message
    return fail(NF4S_ERR_INVALID_ARGUMENT, "layer %u: src len %lld B exceeds slot capacity %lld B",
                layer_idx, (long long)len, (long long)d->capacity);
  const int b = d->staging;
  // The copy into a slot must wait for its last reader; without a release
  // there is nothing to wait for (vram_double_buffer.rs:258-262).
  if (d->held[b])
    return fail(NF4S_ERR_INVALID_ARGUMENT,
                "layer %u: slot still holds layer %u, which was not released", layer_idx,
                d->layer[b]);
  hipError_t e = hipSuccess;
  if (d->freed_valid[b]) e = hipStreamWaitEvent(d->copy, d->freed[b], 0);
  if (e == hipSuccess && len > 0)
    e = hipMemcpyAsync(d->slot[b], src, (size_t)len, hipMemcpyHostToDevice, d->copy);
  if (e == hipSuccess) e = hipEventRecord(d->ready[b], d->copy);
  if (e != hipSuccess) return hip_fail(e, "dbuf_advance");
  d->freed_valid[b] = false;
  d->held[b] = true;
  d->layer[b] = layer_idx;
  d->staging = b ^ 1;  // swap: the filled slot becomes the compute slot
  *dev_ptr = d->slot[b];
  *ready_event = reinterpret_cast<void *>(d->ready[b]);
  return NF4S_OK;
}

// Records that everything enqueued so far on `compute_stream` is the last
// use of the slot at `dev_ptr` (a pointer nf4s_dbuf_advance returned); the
// copy that refills that slot waits for it.
int32_t nf4s_dbuf_release(nf4s_dbuf *d, const void *dev_ptr, void *compute_stream) {
  clear_error();
  if (d == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "dbuf is NULL");
  int i = -1;
  for (int k = 0; k < 2; ++k)
    if (d->slot[k] == dev_ptr) i = k;
  if (i < 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "pointer is not a slot of this buffer");
  if (!d->held[i]) return fail(NF4S_ERR_INVALID_ARGUMENT, "slot was not handed out or is released");
  const hipError_t e = hipEventRecord(d->freed[i], as_stream(compute_stream));
  if (e != hipSuccess) return hip_fail(e, "dbuf_release");
  d->freed_valid[i] = true;
  d->held[i] = false;
  return NF4S_OK;
}

// FlowCast::take_ready with the cuda-double-buffer feature
// (flowcast/src/lib.rs:458-498): the pinned bytes of layer `layer_idx` are
// copied into the staging slot on the copy stream, and the ReadyLayer names
// the slot as slab 0 with the copy's event (ready.rs:20-52).
int32_t nf4s_take_ready(nf4s_dbuf *d, uint32_t layer_idx, const void *pinned, int64_t len,
                        nf4s_ready_layer *out) {
  clear_error();
  if (out == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "ReadyLayer is NULL");
  void *ptr = nullptr, *ev = nullptr;
  const int32_t rc = nf4s_dbuf_advance(d, layer_idx, pinned, len, &ptr, &ev);
  if (rc != NF4S_OK) return rc;
  out->layer_idx = layer_idx;
  out->slab_device_ptr = ptr;
  out->bytes = len;
  out->copy_event = ev;
  out->precision = NF4S_PRECISION_NF4;
  out->needs_decode = 0;
  return NF4S_OK;
}

int32_t nf4s_residency_create(uint32_t num_layers, nf4s_residency **out) {
  clear_error();
  if (out == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "out is NULL");
  *out = nullptr;
  try {
    nf4s_residency *r = new nf4s_residency();
    r->layers.resize(num_layers);
    *out = r;
  } catch (...) {
    return fail(NF4S_ERR_INVALID_ARGUMENT, "out of host memory");
  }
  return NF4S_OK;
}

int32_t nf4s_residency_destroy(nf4s_residency *r) {
  clear_error();
  delete r;
  return NF4S_OK;
}

int32_t nf4s_residency_publish(nf4s_residency *r, uint32_t layer_idx, const void *pinned,
                               int64_t bytes, int32_t precision) {
  clear_error();
  if (r == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "residency is NULL");
  if (bytes < 0 || (bytes > 0 && pinned == nullptr))
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad blob for layer %u", layer_idx);
  if (precision < NF4S_PRECISION_FP32 || precision > NF4S_PRECISION_NF4)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "unknown precision %d", precision);
  {
    std::lock_guard<std::mutex> lock(r->mu);
    if (layer_idx >= r->layers.size())
      return fail(NF4S_ERR_LAYER_NOT_FOUND, "layer %u beyond the %zu the table holds", layer_idx,
                  r->layers.size());
    nf4s_residency::Entry &e = r->layers[layer_idx];
    if (e.resident) return fail(NF4S_ERR_INVALID_ARGUMENT, "layer %u is already resident", layer_idx);
    e.resident = true;
    e.pinned = pinned;
    e.bytes = bytes;
    e.precision = precision;
  }
  r->cv.notify_all();
  return NF4S_OK;
}

// state_machine.rs:306-324: the deadline is tested first on every pass,
// then readiness; a ready layer is taken (removed from the map).
int32_t nf4s_residency_wait(nf4s_residency *r, uint32_t layer_idx, int64_t timeout_us,
                            const void **pinned, int64_t *bytes, int32_t *precision) {
  clear_error();
  if (r == nullptr || pinned == nullptr || bytes == nullptr || precision == nullptr)
    return fail(NF4S_ERR_INVALID_ARGUMENT, "bad residency_wait args");
  if (timeout_us < 0) return fail(NF4S_ERR_INVALID_ARGUMENT, "negative timeout");
  // steady_clock counts int64 nanoseconds: longer timeouts (about 31 years
  // and up) wait as long as 10^15 us, so the deadline cannot overflow.
  constexpr int64_t kMaxTimeoutUs = (int64_t)1000000000000000;
  if (timeout_us > kMaxTimeoutUs) timeout_us = kMaxTimeoutUs;
  using clock = std::chrono::steady_clock;
  const clock::time_point start = clock::now();
  const clock::time_point deadline = start + std::chrono::microseconds(timeout_us);
  std::unique_lock<std::mutex> lock(r->mu);
  if (layer_idx >= r->layers.size())
    return fail(NF4S_ERR_LAYER_NOT_FOUND, "layer %u beyond the %zu the table holds", layer_idx,
                r->layers.size());
  for (;;) {
    if (clock::now() >= deadline)
      return fail(NF4S_ERR_PREFETCH_MISS, "prefetch miss on layer %u", layer_idx);
    nf4s_residency::Entry &e = r->layers[layer_idx];
    if (e.resident) {
      e.resident = false;
      *pinned = e.pinned;
      *bytes = e.bytes;
      *precision = e.precision;
      return NF4S_OK;
    }
    r->cv.wait_until(lock, deadline);
  }
}

int32_t nf4s_take_ready_wait(nf4s_dbuf *d, nf4s_residency *r, uint32_t layer_idx,
                             int64_t timeout_us, nf4s_ready_layer *out) {
  clear_error();
  if (d == nullptr || out == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad take_ready args");
  const void *pinned = nullptr;
  int64_t bytes = 0;
  int32_t precision = 0;
  int32_t rc = nf4s_residency_wait(r, layer_idx, timeout_us, &pinned, &bytes, &precision);
  if (rc != NF4S_OK) return rc;
  rc = nf4s_take_ready(d, layer_idx, pinned, bytes, out);
  if (rc != NF4S_OK) return rc;
  out->precision = precision;
  // QuantizedDecoder::needs_decode (flowcast/src/decode.rs:181-183).
  out->needs_decode = (precision == NF4S_PRECISION_INT4 || precision == NF4S_PRECISION_INT8);
  return NF4S_OK;
}

// FlowCast::retire_layer (flowcast/src/lib.rs:543-545): everything enqueued
// so far on `compute_stream` is the layer's last use; the copy that refills
// its slot waits for that.  A ReadyLayer retires once, and only while its
// slot still holds its layer.
int32_t nf4s_retire_layer(nf4s_dbuf *d, const nf4s_ready_layer *layer, void *compute_stream) {
  clear_error();
  if (d == nullptr || layer == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "bad args");
  for (int k = 0; k < 2; ++k)
    if (d->slot[k] == layer->slab_device_ptr && d->held[k] && d->layer[k] != layer->layer_idx)
      return fail(NF4S_ERR_INVALID_ARGUMENT, "layer %u: its slot now holds layer %u",
                  layer->layer_idx, d->layer[k]);
  return nf4s_dbuf_release(d, layer->slab_device_ptr, compute_stream);
}

int32_t nf4s_stream_wait_event(void *stream, void *event) {
  clear_error();
  if (event == nullptr) return fail(NF4S_ERR_INVALID_ARGUMENT, "event is NULL");
  const hipError_t e =
      hipStreamWaitEvent(as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0);
  if (e != hipSuccess) return hip_fail(e, "stream_wait_event");
  return NF4S_OK;
}

}  // extern "C"
