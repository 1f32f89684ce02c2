// Host-to-device transfer lane: the slot-mapping upload path of the
// reference's native cache owner (PagedKVCache::copy_slots_async,
// csrc/paged_kv/paged_kv.cpp:101-168), as a small HIP runtime object.
//
// A lane owns one non-blocking transfer stream (default priority) and
// recycled events.  Each copy is ordered after everything already enqueued
// on the caller's compute stream (so the destination may be a reused
// buffer the compute stream is still reading), and the compute stream waits
// for the copy before any later work.  Copies run in order on the transfer
// stream, so completion is tracked with increasing tickets: the caller keeps
// the pinned source alive until nkv_transfer_poll reports its ticket done.
#include <deque>
#include <mutex>
#include <vector>

#include "nkv_common.h"

struct nkv_transfer {
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t reuse_ready = nullptr;
  hipEvent_t transfer_done = nullptr;
  std::deque<std::pair<int64_t, hipEvent_t>> pending;
  std::vector<hipEvent_t> spare;
  int64_t next_ticket = 1;
  int64_t completed = 0;
  std::mutex mutex;
};

namespace {

// Makes `device` current for the scope and restores the previous device.
class DeviceScope {
 public:
  explicit DeviceScope(int device) {
    if (hipGetDevice(&previous_) != hipSuccess) previous_ = -1;
    if (previous_ != device) status_ = hipSetDevice(device);
  }
  ~DeviceScope() {
    if (previous_ >= 0) (void)hipSetDevice(previous_);
  }
  hipError_t status() const { return status_; }

 private:
  int previous_ = -1;
  hipError_t status_ = hipSuccess;
};

int hip_fail(const char* what, hipError_t err) {
  return nkv_fail(NKV_E_HIP, "%s: %s (%d)", what, hipGetErrorString(err),
                  static_cast<int>(err));
}

// Pops finished copies (in order) and recycles their events.
int release_completed(nkv_transfer* t) {
  while (!t->pending.empty()) {
    const hipError_t st = hipEventQuery(t->pending.front().second);
    if (st == hipErrorNotReady) return NKV_OK;
    if (st != hipSuccess) return hip_fail("nkv_transfer: event query", st);
    t->completed = t->pending.front().first;
    t->spare.push_back(t->pending.front().second);
    t->pending.pop_front();
  }
  return NKV_OK;
}

}  // namespace

extern "C" int nkv_transfer_create(int32_t device, nkv_transfer** out) {
  if (out == nullptr) return nkv_fail(NKV_E_INVALID, "nkv_transfer_create: null output");
  *out = nullptr;
  int count = 0;
  if (hipError_t err = hipGetDeviceCount(&count); err != hipSuccess) {
    return hip_fail("nkv_transfer_create: device count", err);
  }
  if (device < 0 || device >= count) {
    return nkv_fail(NKV_E_INVALID, "nkv_transfer_create: device %d outside [0, %d)",
                    device, count);
  }
  DeviceScope scope(device);
  if (scope.status() != hipSuccess) return hip_fail("nkv_transfer_create: set device", scope.status());
  auto* t = new nkv_transfer();
  t->device = device;
  hipError_t err = hipStreamCreateWithFlags(&t->stream, hipStreamNonBlocking);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&t->reuse_ready, hipEventDisableTiming);
  if (err == hipSuccess) err = hipEventCreateWithFlags(&t->transfer_done, hipEventDisableTiming);
  if (err != hipSuccess) {
    if (t->transfer_done) (void)hipEventDestroy(t->transfer_done);
    if (t->reuse_ready) (void)hipEventDestroy(t->reuse_ready);
    if (t->stream) (void)hipStreamDestroy(t->stream);
    delete t;
    return hip_fail("nkv_transfer_create", err);
  }
  *out = t;
  return NKV_OK;
}

extern "C" int nkv_transfer_destroy(nkv_transfer* t) {
  if (t == nullptr) return NKV_OK;
  DeviceScope scope(t->device);
  int rc = NKV_OK;
  if (hipError_t err = hipStreamSynchronize(t->stream); err != hipSuccess) {
    rc = hip_fail("nkv_transfer_destroy: synchronize", err);
  }
  for (auto& entry : t->pending) (void)hipEventDestroy(entry.second);
  for (hipEvent_t e : t->spare) (void)hipEventDestroy(e);
  (void)hipEventDestroy(t->transfer_done);
  (void)hipEventDestroy(t->reuse_ready);
  (void)hipStreamDestroy(t->stream);
  delete t;
  return rc;
}

extern "C" int nkv_transfer_h2d(nkv_transfer* t, void* dst, const void* src,
                                int64_t bytes, void* compute_stream,
                                int64_t* ticket) {
  if (t == nullptr || ticket == nullptr) {
    return nkv_fail(NKV_E_INVALID, "nkv_transfer_h2d: null lane or ticket");
  }
  if (bytes < 0) return nkv_fail(NKV_E_INVALID, "nkv_transfer_h2d: negative size");
  if (bytes > 0 && (dst == nullptr || src == nullptr)) {
    return nkv_fail(NKV_E_INVALID, "nkv_transfer_h2d: null pointer");
  }
  std::lock_guard<std::mutex> lock(t->mutex);
  DeviceScope scope(t->device);
  if (scope.status() != hipSuccess) return hip_fail("nkv_transfer_h2d: set device", scope.status());
  if (int rc = release_completed(t)) return rc;
  auto compute = static_cast<hipStream_t>(compute_stream);
  hipEvent_t done = nullptr;
  if (!t->spare.empty()) {
    done = t->spare.back();
    t->spare.pop_back();
  } else if (hipError_t err = hipEventCreateWithFlags(&done, hipEventDisableTiming);
             err != hipSuccess) {
    return hip_fail("nkv_transfer_h2d: event create", err);
  }
  hipError_t err = hipEventRecord(t->reuse_ready, compute);
  if (err == hipSuccess) err = hipStreamWaitEvent(t->stream, t->reuse_ready, 0);
  if (err == hipSuccess && bytes > 0) {
    err = hipMemcpyAsync(dst, src, static_cast<size_t>(bytes), hipMemcpyHostToDevice, t->stream);
  }
  if (err == hipSuccess) err = hipEventRecord(done, t->stream);
  if (err == hipSuccess) err = hipEventRecord(t->transfer_done, t->stream);
  if (err == hipSuccess) err = hipStreamWaitEvent(compute, t->transfer_done, 0);
  if (err != hipSuccess) {
    t->spare.push_back(done);
    return hip_fail("nkv_transfer_h2d", err);
  }
  *ticket = t->next_ticket++;
  t->pending.emplace_back(*ticket, done);
  return NKV_OK;
}

extern "C" int nkv_transfer_poll(nkv_transfer* t, int64_t* in_flight,
                                 int64_t* completed_upto) {
  if (t == nullptr) return nkv_fail(NKV_E_INVALID, "nkv_transfer_poll: null lane");
  std::lock_guard<std::mutex> lock(t->mutex);
  DeviceScope scope(t->device);
  if (int rc = release_completed(t)) return rc;
  if (in_flight) *in_flight = static_cast<int64_t>(t->pending.size());
  if (completed_upto) *completed_upto = t->completed;
  return NKV_OK;
}

extern "C" int nkv_transfer_synchronize(nkv_transfer* t) {
  if (t == nullptr) return nkv_fail(NKV_E_INVALID, "nkv_transfer_synchronize: null lane");
  std::lock_guard<std::mutex> lock(t->mutex);
  DeviceScope scope(t->device);
  if (hipError_t err = hipStreamSynchronize(t->stream); err != hipSuccess) {
    return hip_fail("nkv_transfer_synchronize", err);
  }
  return release_completed(t);
}
