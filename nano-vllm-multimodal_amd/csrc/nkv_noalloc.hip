// Varlen K/V gather for callers that cannot allocate device memory (code
// under HIP graph capture, serving loops that forbid hipMalloc).
//
// nkv_gather_varlen needs a plan buffer of 16 bytes per chunk, which the
// caller passes as a workspace.  This entry point keeps that plan in a
// file-scope device array instead, so the call allocates nothing: the array
// is part of the library's code object, one copy per GPU, loaded with the
// module and held until the process ends.
//
// In host code `scratch` names a host-side shadow, not the device array, so
// it is never passed to a kernel or a HIP copy.  The device address is
// looked up once per device with hipGetSymbolAddress (on the first call made
// with that device current) and cached; every later use goes through that
// pointer.  All calls on one GPU share its array, and the array keeps the
// last call's plan: calls that overlap on one GPU (different streams, or
// threads without ordering between them) race on it.  Calls on one stream
// are ordered by the stream and never overlap.  The plan builder writes every
// entry the gather reads, so nothing needs to be cleared between calls.
#include <atomic>
#include <mutex>

#include "nkv_common.h"

namespace nkv {
namespace {

static __device__ __align__(256) uint8_t scratch[NKV_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_address[kMaxDevices];
std::mutex g_scratch_lookup;

// Device address of the current device's `scratch` array (looked up once per
// device, then cached).
int scratch_address(void** out) {
  int device = -1;
  hipError_t err = hipGetDevice(&device);
  if (err != hipSuccess) {
    return nkv_fail(NKV_E_HIP, "nkv_gather_varlen_noalloc: hipGetDevice failed: %s",
                    hipGetErrorString(err));
  }
  if (device < 0 || device >= kMaxDevices) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_noalloc: device %d beyond %d devices",
                    device, kMaxDevices);
  }
  void* address = g_scratch_address[device].load(std::memory_order_acquire);
  if (address == nullptr) {
    std::lock_guard<std::mutex> lock(g_scratch_lookup);
    address = g_scratch_address[device].load(std::memory_order_relaxed);
    if (address == nullptr) {
      err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
      if (err != hipSuccess || address == nullptr) {
        return nkv_fail(NKV_E_HIP,
                        "nkv_gather_varlen_noalloc: hipGetSymbolAddress(scratch) "
                        "failed on device %d: %s",
                        device, hipGetErrorString(err));
      }
      g_scratch_address[device].store(address, std::memory_order_release);
    }
  }
  *out = address;
  return NKV_OK;
}

}  // namespace
}  // namespace nkv

extern "C" int nkv_gather_varlen_noalloc(
    const void* key_cache, const void* value_cache, const int32_t* block_tables,
    int64_t table_stride, const int32_t* cu_seqlens_k, int64_t num_seqs,
    int64_t total_rows, int64_t block_size, int64_t row_elems,
    int64_t num_blocks, int32_t dtype, void* key_out, void* value_out,
    void* stream) {
  if (total_rows < 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_noalloc: total_rows must be non-negative");
  }
  if (total_rows == 0) return NKV_OK;
  const int64_t capacity =
      nkv_gather_plan_capacity(total_rows, num_seqs, block_size, row_elems, dtype);
  if (capacity <= 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_noalloc: bad geometry");
  }
  // Checked before the device is touched: the plan must fit the array.
  if (capacity > NKV_SCRATCH_BYTES / 16) {
    return nkv_fail(NKV_E_CAPACITY,
                    "nkv_gather_varlen_noalloc: the plan needs %lld bytes, more than "
                    "the library's %d-byte scratch (use nkv_gather_varlen with a "
                    "workspace)",
                    static_cast<long long>(capacity * 16), NKV_SCRATCH_BYTES);
  }
  void* plan = nullptr;
  if (int rc = nkv::scratch_address(&plan)) return rc;
  if (int rc = nkv_build_gather_plan(block_tables, table_stride, cu_seqlens_k,
                                     num_seqs, total_rows, block_size,
                                     row_elems, num_blocks, dtype, plan,
                                     capacity, stream)) {
    return rc;
  }
  return nkv_gather_varlen_planned(key_cache, value_cache, plan, capacity,
                                   num_blocks * block_size, total_rows,
                                   block_size, row_elems, dtype, key_out,
                                   value_out, stream);
}
