// Paged KV store: scatter per-token K/V rows into the paged caches.
//
// Semantics follow the reference pytorch backend
// (nanovllm/layers/paged_kv/pytorch_backend.py:26-38): rows whose slot is -1
// are skipped, every other row t lands in cache row slot_mapping[t]
// (row = one (block, in-block slot) pair of the [num_blocks, block_size,
// kv_heads, head_dim] cache).  K and V are moved in the same pass.
//
// Mapping: one 64-lane wavefront per group of rows.  A row of row_words
// words is walked by lanes_per_row = min(64, pow2ceil(row_words)) lanes, so
// a 2 KiB bf16 row (8 kv heads x 128) is one wavefront issuing 2 K and 2 V
// 16-byte loads per lane before any store, and a 512 B row (2 x 128) puts two
// rows in one wavefront.  The work is pure bandwidth (no MFMA, no LDS).
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kStoreThreads = 256;
constexpr int kStoreMaxBlocks = 16384;

template <int W>
__global__ __launch_bounds__(kStoreThreads) void store_rows_kernel(
    const uint8_t* __restrict__ key, const uint8_t* __restrict__ value,
    uint8_t* __restrict__ key_cache, uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ slot_mapping, int32_t num_tokens,
    int64_t key_stride, int64_t value_stride, int64_t row_bytes,
    int32_t row_words, int32_t lpr_shift, int64_t num_slots) {
  using T = typename Word<W>::type;
  const int32_t lane = threadIdx.x & (kWave - 1);
  const int32_t lanes_per_row = 1 << lpr_shift;
  const int32_t rows_per_wave = kWave >> lpr_shift;
  const int32_t col0 = lane & (lanes_per_row - 1);
  const int32_t sub = lane >> lpr_shift;
  const int32_t wave = (blockIdx.x * kStoreThreads + threadIdx.x) / kWave;
  const int32_t num_waves = (gridDim.x * kStoreThreads) / kWave;
  for (int32_t t = wave * rows_per_wave + sub; t < num_tokens;
       t += num_waves * rows_per_wave) {
    const int32_t slot = slot_mapping[t];
    if (slot < 0 || slot >= num_slots) continue;  // -1 padding (and garbage)
    const T* ks = reinterpret_cast<const T*>(key + t * key_stride);
    const T* vs = reinterpret_cast<const T*>(value + t * value_stride);
    T* kd = reinterpret_cast<T*>(key_cache + slot * row_bytes);
    T* vd = reinterpret_cast<T*>(value_cache + slot * row_bytes);
    for (int32_t c = col0; c < row_words; c += 2 * lanes_per_row) {
      const int32_t c1 = c + lanes_per_row;
      const bool two = c1 < row_words;
      const T k0 = ks[c];
      const T v0 = vs[c];
      T k1{}, v1{};
      if (two) {
        k1 = ks[c1];
        v1 = vs[c1];
      }
      kd[c] = k0;
      vd[c] = v0;
      if (two) {
        kd[c1] = k1;
        vd[c1] = v1;
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
  int lpr_shift = 0;
  while ((int64_t{1} << lpr_shift) < row_words && lpr_shift < 6) ++lpr_shift;
  const int64_t rows_per_wave = kWave >> lpr_shift;
  const int64_t waves = (num_tokens + rows_per_wave - 1) / rows_per_wave;
  const int64_t waves_per_block = kStoreThreads / kWave;
  int64_t blocks = (waves + waves_per_block - 1) / waves_per_block;
  if (blocks > kStoreMaxBlocks) blocks = kStoreMaxBlocks;
  store_rows_kernel<W><<<dim3(static_cast<unsigned>(blocks)),
                         dim3(kStoreThreads), 0, stream>>>(
      static_cast<const uint8_t*>(key), static_cast<const uint8_t*>(value),
      static_cast<uint8_t*>(key_cache), static_cast<uint8_t*>(value_cache),
      slots, num_tokens, ks, vs, row_bytes, static_cast<int32_t>(row_words),
      lpr_shift, num_slots);
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
