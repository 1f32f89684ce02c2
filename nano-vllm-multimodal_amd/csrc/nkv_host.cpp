// Per-call host path of the hip backend's store and gather.
//
// The reference's SDPA decode calls its backend's gather twice per request
// per layer (nanovllm/layers/attention.py:284-300) and its store once per
// layer (attention.py:87-93).  Each call validates its inputs
// (nanovllm/layers/paged_kv/base.py:75-151) and launches one kernel.  On
// MI355X the launch alone costs about 3 us of host time, so Python around
// it (argument checks, the output allocation, a ctypes call) was most of a
// call.  This module runs the same checks, in the same order and with the
// same ValueError messages as nanokv.paged_kv.base.check_store_inputs /
// check_gather_inputs, allocates the gather's output with torch's caching
// allocator, and calls the library's C ABI (include/nanokv.h) directly.
//
// torch is plumbing here: it unpacks the tensors and allocates; every byte
// is moved by the HIP library.  The module does not link libnanokv.so: the
// Python loader hands it the entry points of the library it loaded, so a
// library chosen at run time is the one that runs.  The stream is the
// caller's current stream, passed in as a hipStream_t integer.
#include <torch/extension.h>

#include <cctype>
#include <cstdint>
#include <cstdlib>
#include <string>

#include "nanokv.h"

#ifndef NKV_HOST_BUILD_ID
#define NKV_HOST_BUILD_ID "unfingerprinted"
#endif

namespace {

namespace py = pybind11;

using StoreFn = int (*)(const void*, const void*, void*, void*, const int32_t*, int64_t, int64_t,
                        int64_t, int64_t, int64_t, int32_t, void*);
using GatherFn = int (*)(const void*, const int32_t*, int64_t, int64_t, int64_t, int64_t, int64_t,
                         int32_t, void*, void*);
using LastErrorFn = const char* (*)();

StoreFn g_store = nullptr;
GatherFn g_gather = nullptr;
LastErrorFn g_last_error = nullptr;

[[noreturn]] void value_error(const std::string& what) { throw py::value_error(what); }

void require_bound() {
  if (g_store == nullptr || g_gather == nullptr || g_last_error == nullptr) {
    throw std::runtime_error("nanokv host path: bind() the library's entry points first");
  }
}

// base.py:68-72: index values in host memory are always range-checked;
// device-resident ones only when NANOVLLM_PAGED_KV_VALIDATE_INDICES is one
// of 1 / true / yes / on (read on every call, as the reference does).
bool index_values_checked(const at::Tensor& t) {
  if (!t.is_cuda()) return true;
  const char* raw = std::getenv("NANOVLLM_PAGED_KV_VALIDATE_INDICES");
  std::string flag = raw != nullptr ? raw : "0";
  const char* space = " \t\n\r\f\v";
  const size_t first = flag.find_first_not_of(space);
  flag = first == std::string::npos ? "" : flag.substr(first, flag.find_last_not_of(space) - first + 1);
  for (char& c : flag) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
  return flag == "1" || flag == "true" || flag == "yes" || flag == "on";
}

int32_t dtype_code(at::ScalarType type) {
  switch (type) {
    case at::kHalf:
      return NKV_DTYPE_FLOAT16;
    case at::kBFloat16:
      return NKV_DTYPE_BFLOAT16;
    case at::kFloat:
      return NKV_DTYPE_FLOAT32;
    default:
      throw std::runtime_error(std::string("nanokv paged KV ops support float16, bfloat16 and "
                                           "float32, not ") + c10::toString(type));
  }
}

void check_status(int status, const char* what) {
  if (status != 0) {
    throw std::runtime_error(std::string(what) + " failed (nkv status " + std::to_string(status) +
                             "): " + g_last_error());
  }
}

// The checks of base.py:75-114 (nanokv.paged_kv.base.check_store_inputs).
void check_store(const at::Tensor& key, const at::Tensor& value, const at::Tensor& key_cache,
                 const at::Tensor& value_cache, const at::Tensor& slot_mapping) {
  if (key.dim() != 3 || value.dim() != 3 || key.sizes() != value.sizes()) {
    value_error("key and value must have matching shape [tokens, kv_heads, head_dim]");
  }
  if (key.stride(-1) != 1 || value.stride(-1) != 1) {
    value_error("key and value inner dimensions must be contiguous");
  }
  if (key_cache.dim() != 4 || value_cache.dim() != 4 || key_cache.sizes() != value_cache.sizes()) {
    value_error("key and value cache shape must match [blocks, block, kv_heads, head_dim]");
  }
  if (key_cache.size(2) != key.size(1) || key_cache.size(3) != key.size(2)) {
    value_error("cache shape does not match key/value kv_heads and head_dim");
  }
  const at::Device device = key.device();
  if (value.device() != device || key_cache.device() != device || value_cache.device() != device ||
      slot_mapping.device() != device) {
    value_error("all paged KV Store tensors must be on the same device");
  }
  const at::ScalarType type = key.scalar_type();
  if (value.scalar_type() != type || key_cache.scalar_type() != type ||
      value_cache.scalar_type() != type) {
    value_error("key, value, and caches must have matching dtype");
  }
  if (slot_mapping.scalar_type() != at::kInt || slot_mapping.dim() != 1) {
    value_error("slot_mapping must be a one-dimensional int32 tensor");
  }
  if (slot_mapping.size(0) != key.size(0)) {
    value_error("slot_mapping length must equal the number of input tokens");
  }
  if (!slot_mapping.is_contiguous()) value_error("slot_mapping must be contiguous");
  if (key.size(0) > 0 && index_values_checked(slot_mapping)) {
    const int64_t num_slots = key_cache.size(0) * key_cache.size(1);
    if (((slot_mapping < -1) | (slot_mapping >= num_slots)).any().item<bool>()) {
      value_error("slot_mapping contains a slot outside [-1, " + std::to_string(num_slots) + ")");
    }
  }
}

// The checks of base.py:117-151 (nanokv.paged_kv.base.check_gather_inputs).
void check_gather(const at::Tensor& cache, const at::Tensor& table, int64_t sequence_length) {
  if (cache.dim() != 4) value_error("cache must have shape [blocks, block, kv_heads, head_dim]");
  if (cache.stride(-1) != 1) value_error("cache inner dimensions must be contiguous");
  if (table.scalar_type() != at::kInt || table.dim() != 1) {
    value_error("block_table must be a one-dimensional int32 tensor");
  }
  if (table.device() != cache.device()) {
    value_error("cache and block_table must be on the same device");
  }
  if (!table.is_contiguous()) value_error("block_table must be contiguous");
  if (sequence_length < 0) value_error("sequence_length must be non-negative");
  const int64_t block_size = cache.size(1);
  const int64_t required = (sequence_length + block_size - 1) / block_size;
  if (table.size(0) < required) {
    value_error("block_table does not cover the requested sequence length");
  }
  if (required > 0 && index_values_checked(table)) {
    const at::Tensor used = table.slice(0, 0, required);
    if (((used < 0) | (used >= cache.size(0))).any().item<bool>()) {
      value_error("block_table contains an invalid physical block");
    }
  }
}

void store(const at::Tensor& key_in, const at::Tensor& value_in, const at::Tensor& key_cache,
           const at::Tensor& value_cache, const at::Tensor& slot_mapping, int64_t stream) {
  check_store(key_in, value_in, key_cache, value_cache, slot_mapping);
  if (!key_in.is_cuda()) value_error("HIP Paged KV Store requires ROCm device tensors");
  require_bound();
  if (!key_cache.is_contiguous() || !value_cache.is_contiguous()) {
    value_error("paged KV HIP Store requires contiguous [blocks, block, kv_heads, head_dim] caches");
  }
  const int64_t tokens = key_in.size(0);
  if (tokens == 0) return;
  const int32_t code = dtype_code(key_in.scalar_type());
  // The kernel addresses a token's [kv_heads, head_dim] as one contiguous
  // row through the token stride; a head-strided view is compacted first.
  const bool strided = key_in.size(1) > 1;
  const at::Tensor key =
      strided && key_in.stride(1) != key_in.size(2) ? key_in.contiguous() : key_in;
  const at::Tensor value =
      strided && value_in.stride(1) != value_in.size(2) ? value_in.contiguous() : value_in;
  check_status(g_store(key.data_ptr(), value.data_ptr(), key_cache.data_ptr(),
                       value_cache.data_ptr(), slot_mapping.data_ptr<int32_t>(), tokens,
                       key.stride(0), value.stride(0), key.size(1) * key.size(2),
                       key_cache.size(0) * key_cache.size(1), code,
                       reinterpret_cast<void*>(stream)),
               "nanovllm_paged_kv::store");
}

at::Tensor gather(const at::Tensor& cache, const at::Tensor& table, int64_t sequence_length,
                  int64_t stream) {
  check_gather(cache, table, sequence_length);
  if (!cache.is_cuda()) value_error("HIP Paged KV Gather requires ROCm device tensors");
  require_bound();
  if (!cache.is_contiguous()) {
    value_error("paged KV HIP Gather requires contiguous [blocks, block, kv_heads, head_dim] caches");
  }
  at::Tensor out = at::empty({sequence_length, cache.size(2), cache.size(3)}, cache.options());
  if (sequence_length == 0) return out;
  const int32_t code = dtype_code(cache.scalar_type());
  check_status(g_gather(cache.data_ptr(), table.data_ptr<int32_t>(), table.size(0),
                        sequence_length, cache.size(1), cache.size(2) * cache.size(3),
                        cache.size(0), code, out.data_ptr(), reinterpret_cast<void*>(stream)),
               "nanovllm_paged_kv::gather");
  return out;
}

void bind(uintptr_t store_fn, uintptr_t gather_fn, uintptr_t last_error_fn) {
  g_store = reinterpret_cast<StoreFn>(store_fn);
  g_gather = reinterpret_cast<GatherFn>(gather_fn);
  g_last_error = reinterpret_cast<LastErrorFn>(last_error_fn);
}

}  // namespace

PYBIND11_MODULE(_nkv_host, m) {
  m.doc() = "Per-call host path of the nanokv hip backend's store and gather";
  m.def("bind", &bind, "set the library entry points (nkv_store, nkv_gather, nkv_last_error)");
  m.def("store", &store, "validated store launch on a stream");
  m.def("gather", &gather, "validated gather launch on a stream; returns the new tensor");
  m.def("check_store", &check_store, "the store validator's checks (no launch)");
  m.def("check_gather", &check_gather, "the gather validator's checks (no launch)");
  m.def("build_id", []() { return std::string(NKV_HOST_BUILD_ID); });
}
