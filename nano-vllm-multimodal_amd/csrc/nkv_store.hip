// Paged KV store: scatter per-token K/V rows into the paged caches.
//
// Semantics follow the reference pytorch backend
// (nanovllm/layers/paged_kv/pytorch_backend.py:26-38): rows whose slot is -1
// are skipped, every other row t lands in cache row slot_mapping[t]
// (row = one (block, in-block slot) pair of the [num_blocks, block_size,
// kv_heads, head_dim] cache).  K and V are moved by the same launch.
//
// Launch shape (measured on MI355X with rocprofv3 on the chunked-prefill
// store, 67 MB, and the narrow-row store, 107 MB): short-lived 128-thread
// workgroups, each moving ~4 KiB of ONE tensor (K rows in blockIdx.y == 0,
// V rows in blockIdx.y == 1) in one batch, with non-temporal accesses.  A
// workgroup takes rows_per_wg consecutive tokens (2 rows of 2 KiB, 8 of
// 512 B); consecutive lanes move consecutive words of a row.  Each lane
// issues its data loads together with its slot loads, one memory round
// trip per batch instead of two (-2 to -4%).  Workgroup size (64-512
// threads), bytes per workgroup (2-16 KiB), an XCD-contiguous workgroup
// order and ordinary (cached) stores change the steady-state rate of
// back-to-back stores by under 3%; ordinary stores look up to 10% faster
// when each launch is timed alone after a cache eviction, because the
// 256 MB MALL then absorbs the launch's writes and their write-back falls
// outside it.  The work is pure bandwidth (no MFMA, no LDS).
#include "nkv_common.h"

namespace nkv {
namespace {

#ifndef NKV_STORE_THREADS
#define NKV_STORE_THREADS 128
#endif
#ifndef NKV_STORE_WG_BYTES
#define NKV_STORE_WG_BYTES 4096
#endif

// 1: a lane issues its rows' data loads together with their slot loads (one
// memory round trip per batch; a row whose slot turns out invalid has been
// read for nothing, which only -1 padding rows cost).  0: data loads wait
// for the slots and skip invalid rows.
#ifndef NKV_STORE_SPECULATIVE
#define NKV_STORE_SPECULATIVE 1
#endif

// Cache policy of the K/V reads and of the cache writes (1 = non-temporal).
#ifndef NKV_STORE_NT_LOADS
#define NKV_STORE_NT_LOADS 1
#endif
#ifndef NKV_STORE_NT_STORES
#define NKV_STORE_NT_STORES 1
#endif

template <typename T>
__device__ __forceinline__ T store_src_load(const T* p) {
  if constexpr (NKV_STORE_NT_LOADS) return load_stream(p);
  return *p;
}
template <typename T>
__device__ __forceinline__ void store_dst_store(T* p, T v) {
  if constexpr (NKV_STORE_NT_STORES) {
    store_stream(p, v);
  } else {
    *p = v;
  }
}

constexpr int kStoreThreads = NKV_STORE_THREADS;

// Words per lane issued together: one workgroup's NKV_STORE_WG_BYTES in one
// batch, so a lane waits for memory once per batch instead of once per word.
template <int W>
constexpr int store_batch() {
  return NKV_STORE_WG_BYTES / (W * kStoreThreads) > 0
             ? NKV_STORE_WG_BYTES / (W * kStoreThreads) : 1;
}

template <int W>
__global__ __launch_bounds__(kStoreThreads) void store_rows_kernel(
    const uint8_t* __restrict__ key, const uint8_t* __restrict__ value,
    uint8_t* __restrict__ key_cache, uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ slot_mapping, int32_t num_tokens,
    int64_t key_stride, int64_t value_stride, int64_t row_bytes,
    int32_t row_words, int32_t rows_per_wg, int64_t num_slots) {
  using T = typename Word<W>::type;
  constexpr int U = store_batch<W>();
  const bool second = blockIdx.y != 0;
  const uint8_t* src = second ? value : key;
  const int64_t stride = second ? value_stride : key_stride;
  uint8_t* dst = second ? value_cache : key_cache;
  const int32_t t0 = blockIdx.x * rows_per_wg;  // < num_tokens by the grid
  const int32_t nwords = min(rows_per_wg, num_tokens - t0) * row_words;
  for (int32_t base = 0; base < nwords; base += U * kStoreThreads) {
    int32_t row[U], col[U], slot[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t w = base + u * kStoreThreads + static_cast<int32_t>(threadIdx.x);
      row[u] = w / row_words;
      col[u] = w - row[u] * row_words;
      slot[u] = w < nwords ? slot_mapping[t0 + row[u]] : -1;
    }
    T v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int32_t w = base + u * kStoreThreads + static_cast<int32_t>(threadIdx.x);
      // -1 padding (and any slot outside the cache) is never stored; with
      // NKV_STORE_SPECULATIVE its row is still read (in bounds: t < num_tokens)
      const bool load = NKV_STORE_SPECULATIVE ? w < nwords : (slot[u] >= 0 && slot[u] < num_slots);
      if (load) {
        v[u] = store_src_load(reinterpret_cast<const T*>(src + (t0 + row[u]) * stride) + col[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (slot[u] >= 0 && slot[u] < num_slots) {
        store_dst_store(reinterpret_cast<T*>(dst + slot[u] * row_bytes) + col[u], v[u]);
      }
    }
  }
}

template <int W>
int launch_store(const void* key, const void* value, void* key_cache,
                 void* value_cache, const int32_t* slots, int32_t num_tokens,
                 int64_t ks, int64_t vs, int64_t row_bytes, int64_t num_slots,
                 hipStream_t stream) {
  const int64_t row_words = row_bytes / W;
  int64_t rows_per_wg = NKV_STORE_WG_BYTES / row_bytes;
  if (rows_per_wg < 1) rows_per_wg = 1;
  if (rows_per_wg * row_words > INT32_MAX) rows_per_wg = 1;
  const int64_t blocks = (num_tokens + rows_per_wg - 1) / rows_per_wg;
  store_rows_kernel<W><<<dim3(static_cast<unsigned>(blocks), 2),
                         dim3(kStoreThreads), 0, stream>>>(
      static_cast<const uint8_t*>(key), static_cast<const uint8_t*>(value),
      static_cast<uint8_t*>(key_cache), static_cast<uint8_t*>(value_cache),
      slots, num_tokens, ks, vs, row_bytes, static_cast<int32_t>(row_words),
      static_cast<int32_t>(rows_per_wg), num_slots);
  return nkv_check_launch("nkv_store");
}

}  // namespace
}  // namespace nkv

extern "C" int nkv_store(const void* key, const void* value, void* key_cache,
                         void* value_cache, const int32_t* slot_mapping,
                         int64_t num_tokens, int64_t key_token_stride,
                         int64_t value_token_stride, int64_t row_elems,
                         int64_t num_slots, int32_t dtype, void* stream) {
  using namespace nkv;
  const int eb = element_bytes(dtype);
  if (eb == 0) return nkv_fail(NKV_E_INVALID, "nkv_store: unknown dtype %d", dtype);
  if (num_tokens < 0 || row_elems <= 0 || num_slots < 0 ||
      key_token_stride < 0 || value_token_stride < 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_store: negative size or stride (tokens=%lld row=%lld "
                    "slots=%lld)",
                    static_cast<long long>(num_tokens),
                    static_cast<long long>(row_elems),
                    static_cast<long long>(num_slots));
  }
  if (num_tokens == 0) return NKV_OK;
  if (num_tokens > INT32_MAX || num_slots > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_store: tokens/slots exceed int32");
  }
  if (!key || !value || !key_cache || !value_cache || !slot_mapping) {
    return nkv_fail(NKV_E_INVALID, "nkv_store: null pointer");
  }
  const int64_t row_bytes = row_elems * eb;
  const int64_t ks = key_token_stride * eb;
  const int64_t vs = value_token_stride * eb;
  const int w = common_word_bytes(
      {reinterpret_cast<uint64_t>(key), reinterpret_cast<uint64_t>(value),
       reinterpret_cast<uint64_t>(key_cache),
       reinterpret_cast<uint64_t>(value_cache), static_cast<uint64_t>(ks),
       static_cast<uint64_t>(vs), static_cast<uint64_t>(row_bytes)});
  if (row_bytes / w > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_store: row too large");
  }
  const auto n = static_cast<int32_t>(num_tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (w) {
    case 16:
      return launch_store<16>(key, value, key_cache, value_cache, slot_mapping,
                              n, ks, vs, row_bytes, num_slots, s);
    case 8:
      return launch_store<8>(key, value, key_cache, value_cache, slot_mapping,
                             n, ks, vs, row_bytes, num_slots, s);
    case 4:
      return launch_store<4>(key, value, key_cache, value_cache, slot_mapping,
                             n, ks, vs, row_bytes, num_slots, s);
    case 2:
      return launch_store<2>(key, value, key_cache, value_cache, slot_mapping,
                             n, ks, vs, row_bytes, num_slots, s);
    default:
      return nkv_fail(NKV_E_INVALID,
                      "nkv_store: pointers/strides not aligned to the element "
                      "size");
  }
}
