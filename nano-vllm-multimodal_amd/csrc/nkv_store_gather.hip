// Prefill store + context gather in one launch.
//
// The reference's SDPA prefill stores the layer's new K/V rows into the
// paged cache (nanovllm/layers/attention.py:87-93), then gathers every
// request's whole context back out of the cache (attention.py:250-259,
// the per-request gather of cu_seqlens_k lengths).  The new rows of a
// request are the last ones of its context: request i has
// Lq = cu_seqlens_q[i+1] - cu_seqlens_q[i] new tokens at context positions
// [Lk - Lq, Lk), Lk = cu_seqlens_k[i+1] - cu_seqlens_k[i], and token t of
// the batch sits at position Lk - Lq + (t - cu_seqlens_q[i]), whose cache
// slot is block_tables[i][p / block_size] * block_size + p % block_size.
//
// One launch does both steps with each byte moved once:
//  * new-row workgroups read a token's K (or V) row once and write it to
//    its cache slot (the store) and to its context row of the gathered
//    output (the gather);
//  * cached-row workgroups copy the cached prefixes, positions [0, Lk - Lq),
//    from the cache to the output, driven by chunk entries exactly as the
//    varlen gather's plan drives its copies.
// That is what store followed by gather produces whenever every token's
// slot is -1 or the table-derived slot of its position and no slot repeats,
// which is how the reference packs them (model_runner.py:757-820) and what
// its store already requires (duplicate slots are an upstream contract,
// attention.py:24-25).  A token whose slot is -1 (or differs from its
// table-derived slot) is stored as given, and its output row is read from
// the cache row of its position instead, as the gather would find it.
//
// No cached-prefix row is written in the same step.  A request's cached
// prefix is either its own earlier chunks or blocks it hit in the prefix
// cache, and a block enters the prefix cache only after the step that
// filled it: Scheduler.postprocess calls BlockManager.hash_blocks once the
// model has run (nanovllm/engine/scheduler.py:196-200), hash_blocks is the
// one place a hash is registered (block_manager.py:229-258), and
// can_allocate / allocate only look hashes up (block_manager.py:119-198).
// So the cached-row copies and the new-row stores of one launch touch
// disjoint cache rows, and the two kinds of workgroups need no ordering.  A
// batch that breaks this (a request reading, as cached prefix, rows another
// request of the same call stores) gets unspecified values in those output
// rows, never an access outside the buffers; store then gather handles it.
//
// The plan (one launch per step, shared by all layers and by K and V):
//  * per token t, {output row, table-derived slot} (-1 where there is none);
//  * per chunk of a cached prefix, {source row, output row, rows, request},
//    the varlen gather's entry layout.
// Launch shape and cache policy are those of the store and gather
// (128-thread workgroups of ~4 KiB of one tensor, blockIdx.y = K or V, one
// batch of 16-byte words per lane, non-temporal accesses).
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kSgThreads = 128;
constexpr int kSgWgBytes = 4096;
constexpr int kSgPlanThreads = 1024;

template <int W>
constexpr int sg_batch() {
  return kSgWgBytes / (W * kSgThreads) > 0 ? kSgWgBytes / (W * kSgThreads) : 1;
}

// Largest i in [0, n) with cu[i] <= t, for cu non-decreasing with
// cu[0] <= t < cu[n] (global memory; the request owning token t).
__device__ __forceinline__ int32_t owner_in(const int32_t* __restrict__ cu, int32_t n, int32_t t) {
  int32_t lo = 0, hi = n;
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (cu[mid] <= t) {
      lo = mid;
    } else {
      hi = mid;
    }
  }
  return lo;
}

// The whole plan in one launch: every workgroup rescans the per-request
// chunk counts of the cached prefixes in LDS, then the grid strides over
// the chunk entries and over the tokens.
__global__ __launch_bounds__(kSgPlanThreads) void store_gather_plan_kernel(
    const int32_t* __restrict__ tables, int64_t table_stride,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k, int32_t num_seqs,
    int32_t num_tokens, int32_t block_size, int32_t chunk_rows, int64_t num_blocks,
    int64_t out_rows, int2* __restrict__ meta, int4* __restrict__ entries, int64_t capacity) {
  extern __shared__ int32_t s_mem[];
  int32_t* s_first = s_mem;                 // [num_seqs + 1]
  int32_t* s_tmp = s_first + num_seqs + 1;  // [kSgPlanThreads / 64 + 1]
  lds_exclusive_scan<kSgPlanThreads>(
      num_seqs,
      [&](int32_t i) {
        const int32_t cached = (cu_k[i + 1] - cu_k[i]) - (cu_q[i + 1] - cu_q[i]);
        return cached > 0 ? (cached + chunk_rows - 1) / chunk_rows : 0;
      },
      s_first, s_tmp);
  const int64_t total = s_first[num_seqs];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kSgPlanThreads;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kSgPlanThreads + threadIdx.x;
  for (int64_t k = first; k < capacity; k += stride) {
    int4 entry = make_int4(0, 0, 0, 0);
    if (k < total) {
      const int32_t i = owner_of(s_first, num_seqs, static_cast<int32_t>(k));
      const int32_t row0 = (static_cast<int32_t>(k) - s_first[i]) * chunk_rows;
      const int32_t cached = (cu_k[i + 1] - cu_k[i]) - (cu_q[i + 1] - cu_q[i]);
      int64_t nrows = min(chunk_rows, cached - row0);
      const int64_t dst = static_cast<int64_t>(cu_k[i]) + row0;
      if (dst < 0 || dst >= out_rows) nrows = 0;
      if (dst + nrows > out_rows) nrows = out_rows - dst;
      const int64_t logical = row0 / block_size;
      int32_t src = -1;
      if (logical < table_stride) {
        const int32_t block = tables[i * table_stride + logical];
        if (block >= 0 && block < num_blocks) src = block * block_size + row0 % block_size;
      }
      entry = make_int4(src, static_cast<int32_t>(dst), static_cast<int32_t>(nrows), i);
    }
    entries[k] = entry;
  }
  for (int64_t e = first; e < num_tokens; e += stride) {
    const int32_t t = static_cast<int32_t>(e);
    int2 m = make_int2(-1, -1);
    if (num_seqs > 0 && t >= cu_q[0] && t < cu_q[num_seqs]) {
      const int32_t i = owner_in(cu_q, num_seqs, t);
      const int32_t q0 = cu_q[i];
      const int32_t lk = cu_k[i + 1] - cu_k[i];
      const int32_t p = lk - (cu_q[i + 1] - q0) + (t - q0);
      const int64_t row = static_cast<int64_t>(cu_k[i]) + p;
      if (p >= 0 && p < lk && row >= 0 && row < out_rows) {
        m.x = static_cast<int32_t>(row);
        const int64_t logical = p / block_size;
        if (logical < table_stride) {
          const int32_t block = tables[i * table_stride + logical];
          if (block >= 0 && block < num_blocks) m.y = block * block_size + p % block_size;
        }
      }
    }
    meta[t] = m;
  }
}

// Grid position b holds a cached-row workgroup when
// umulhi(b + 1, spread) > umulhi(b, spread), spread = ceil(C * 2^32 / G) for
// C cached-row workgroups of G (C < G): umulhi(b, spread) counts the cached
// workgroups before b, steps by 0 or 1 and reaches exactly C at b = G, so
// the two kinds are spread evenly over the grid and every index of each
// kind occurs once.  The write-heavy new rows (one read, two writes) and the
// cached copies (one read, one write) then share the launch instead of
// running one after the other.  With no new-row workgroups (C = G) every
// position is cached.  32-bit multiplies only (two scalar mul_hi per
// workgroup), no division.
__device__ __forceinline__ bool sg_is_cached(uint32_t b, uint32_t spread, int32_t new_wgs,
                                             uint32_t* index) {
  if (new_wgs == 0) {
    *index = b;
    return true;
  }
  const uint32_t before = __umulhi(b, spread);
  if (__umulhi(b + 1, spread) > before) {
    *index = before;
    return true;
  }
  *index = b - before;
  return false;
}

// Every index read from device memory is re-checked against the buffers
// (slots against num_slots, output rows against out_rows, chunk sources
// against the cache), so no plan can make the launch leave them.
template <int W>
__global__ __launch_bounds__(kSgThreads) void store_gather_kernel(
    const uint8_t* __restrict__ key, const uint8_t* __restrict__ value,
    uint8_t* __restrict__ key_cache, uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ slot_mapping, const int2* __restrict__ meta,
    int32_t num_tokens, int64_t key_stride, int64_t value_stride, int64_t row_bytes,
    int32_t row_words, int32_t rows_per_wg, int64_t num_slots, int32_t new_wgs, uint32_t spread,
    const int4* __restrict__ entries, int32_t subs_per_entry, int32_t sub_rows,
    int64_t out_rows, uint8_t* __restrict__ key_out, uint8_t* __restrict__ value_out) {
  using T = typename Word<W>::type;
  const bool second = blockIdx.y != 0;
  uint8_t* const cache = second ? value_cache : key_cache;
  uint8_t* const out = second ? value_out : key_out;
  uint32_t x;
  if (!sg_is_cached(blockIdx.x, spread, new_wgs, &x)) {
    const uint8_t* const src = second ? value : key;
    const int64_t stride = second ? value_stride : key_stride;
    constexpr int U = sg_batch<W>();
    // x < new_wgs, so t0 < num_tokens by the grid
    const int32_t t0 = static_cast<int32_t>(x) * rows_per_wg;
    const int32_t nwords = min(rows_per_wg, num_tokens - t0) * row_words;
    for (int32_t base = 0; base < nwords; base += U * kSgThreads) {
      int32_t row[U], col[U], slot[U];
      int2 m[U];
      T v[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int32_t w = base + u * kSgThreads + static_cast<int32_t>(threadIdx.x);
        row[u] = w / row_words;
        col[u] = w - row[u] * row_words;
        slot[u] = -1;
        m[u] = make_int2(-1, -1);
        if (w < nwords) {  // slot, plan row and data issue together
          slot[u] = slot_mapping[t0 + row[u]];
          m[u] = meta[t0 + row[u]];
          v[u] = load_stream(reinterpret_cast<const T*>(src + (t0 + row[u]) * stride) + col[u]);
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool stored = slot[u] >= 0 && slot[u] < num_slots;
        if (stored) store_stream(reinterpret_cast<T*>(cache + slot[u] * row_bytes) + col[u], v[u]);
        if (m[u].x >= 0 && m[u].x < out_rows) {
          T o = v[u];
          if (!stored || slot[u] != m[u].y) {
            // not stored at its own position: the gather reads the cache there
            o = T{};
            if (m[u].y >= 0 && m[u].y < num_slots) {
              o = load_stream(reinterpret_cast<const T*>(cache + m[u].y * row_bytes) + col[u]);
            }
          }
          store_stream(reinterpret_cast<T*>(out + m[u].x * row_bytes) + col[u], o);
        }
      }
    }
    return;
  }
  const int32_t e = static_cast<int32_t>(x) / subs_per_entry;
  const int32_t row_off = (static_cast<int32_t>(x) - e * subs_per_entry) * sub_rows;
  const int4 entry = entries[e];
  if (entry.z <= row_off || entry.y < 0 || static_cast<int64_t>(entry.y) + entry.z > out_rows) return;
  const int32_t nrows = min(sub_rows, entry.z - row_off);
  T* d = reinterpret_cast<T*>(out + (static_cast<int64_t>(entry.y) + row_off) * row_bytes);
  const auto nwords = static_cast<int32_t>(nrows * row_bytes / W);
  if (entry.x < 0 || static_cast<int64_t>(entry.x) + entry.z > num_slots) {
    for (int32_t i = threadIdx.x; i < nwords; i += kSgThreads) store_stream(d + i, T{});
    return;
  }
  const T* s = reinterpret_cast<const T*>(cache + (static_cast<int64_t>(entry.x) + row_off) * row_bytes);
  for (int32_t i = threadIdx.x; i < nwords; i += kSgThreads) store_stream(d + i, load_stream(s + i));
}

// Plan layout: num_tokens int2 meta (rounded up to 16 bytes), then one int4
// per chunk.
int64_t meta_bytes(int64_t num_tokens) { return (num_tokens * 8 + 15) / 16 * 16; }

int64_t divisor_at_most(int64_t rows, int64_t target) {
  if (target < 1) target = 1;
  if (target >= rows) return rows;
  for (int64_t r = target; r > 1; --r) {
    if (rows % r == 0) return r;
  }
  return 1;
}

int check_sg_geometry(const char* what, int64_t num_tokens, int64_t num_seqs, int64_t out_rows,
                      int64_t block_size, int64_t row_elems, int64_t num_blocks, int32_t dtype) {
  const int eb = element_bytes(dtype);
  if (eb == 0) return nkv_fail(NKV_E_INVALID, "%s: unknown dtype %d", what, dtype);
  if (num_tokens < 0 || num_tokens > INT32_MAX || num_seqs < 0 ||
      num_seqs > NKV_MAX_PACK_SEQS || out_rows < 0 || out_rows > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID,
                    "%s: num_tokens/num_seqs/out_rows out of range (num_seqs at most %d)", what,
                    NKV_MAX_PACK_SEQS);
  }
  if (block_size <= 0 || row_elems <= 0 || num_blocks < 0 ||
      num_blocks * block_size > INT32_MAX || block_size * row_elems * eb > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "%s: bad block_size/row_elems/num_blocks", what);
  }
  return NKV_OK;
}

// A plan is laid out for one (num_tokens, out_rows, num_seqs, geometry):
// its size must be the one nkv_store_gather_plan_bytes gives for them, so a
// plan built for other counts is rejected instead of read at the wrong
// offsets.
int check_plan_bytes(const char* what, int64_t plan_bytes, int64_t need) {
  if (need > 0 ? plan_bytes != need : plan_bytes < 0) {
    return nkv_fail(NKV_E_CAPACITY,
                    "%s: plan of %lld bytes, these token/context counts and geometry need "
                    "exactly %lld (build the plan for the same counts)",
                    what, static_cast<long long>(plan_bytes), static_cast<long long>(need));
  }
  return NKV_OK;
}

template <int W>
int launch_store_gather(const void* key, const void* value, void* key_cache, void* value_cache,
                        const int32_t* slots, const int2* meta, int32_t num_tokens, int64_t ks,
                        int64_t vs, int64_t row_bytes, int64_t num_slots, const int4* entries,
                        int64_t capacity, int64_t chunk_rows, int64_t out_rows, void* key_out,
                        void* value_out, hipStream_t stream) {
  const int64_t row_words = row_bytes / W;
  int64_t rows_per_wg = kSgWgBytes / row_bytes;
  if (rows_per_wg < 1) rows_per_wg = 1;
  if (rows_per_wg * row_words > INT32_MAX) rows_per_wg = 1;
  const int64_t new_wgs = (num_tokens + rows_per_wg - 1) / rows_per_wg;
  const int64_t sub_rows = divisor_at_most(chunk_rows, kSgWgBytes / row_bytes);
  const int64_t subs = chunk_rows / sub_rows;
  const int64_t cached_wgs = capacity * subs;
  const int64_t wgs = new_wgs + cached_wgs;
  if (wgs == 0) return NKV_OK;
  if (wgs >= INT32_MAX) return nkv_fail(NKV_E_INVALID, "nkv_store_gather: launch too large");
  // ceil(cached * 2^32 / wgs) < 2^32 whenever new_wgs > 0 (see sg_is_cached)
  const uint32_t spread =
      new_wgs > 0 ? static_cast<uint32_t>(((static_cast<uint64_t>(cached_wgs) << 32) + wgs - 1) /
                                          static_cast<uint64_t>(wgs))
                  : 0u;
  store_gather_kernel<W><<<dim3(static_cast<unsigned>(wgs), 2), dim3(kSgThreads), 0, stream>>>(
      static_cast<const uint8_t*>(key), static_cast<const uint8_t*>(value),
      static_cast<uint8_t*>(key_cache), static_cast<uint8_t*>(value_cache), slots, meta,
      num_tokens, ks, vs, row_bytes, static_cast<int32_t>(row_words),
      static_cast<int32_t>(rows_per_wg), num_slots, static_cast<int32_t>(new_wgs), spread,
      entries, static_cast<int32_t>(subs), static_cast<int32_t>(sub_rows), out_rows,
      static_cast<uint8_t*>(key_out), static_cast<uint8_t*>(value_out));
  return nkv_check_launch("nkv_store_gather");
}

}  // namespace
}  // namespace nkv

extern "C" int64_t nkv_store_gather_plan_bytes(int64_t num_tokens, int64_t total_rows,
                                               int64_t num_seqs, int64_t block_size,
                                               int64_t row_elems, int32_t dtype) {
  if (num_tokens < 0 || total_rows < 0) return 0;
  const int64_t capacity =
      nkv_gather_plan_capacity(total_rows, num_seqs, block_size, row_elems, dtype);
  if (capacity <= 0 && total_rows > 0) return 0;
  return nkv::meta_bytes(num_tokens) + 16 * capacity;
}

extern "C" int nkv_build_store_gather_plan(const int32_t* block_tables, int64_t table_stride,
                                           const int32_t* cu_seqlens_q,
                                           const int32_t* cu_seqlens_k, int64_t num_seqs,
                                           int64_t num_tokens, int64_t out_rows,
                                           int64_t block_size, int64_t row_elems,
                                           int64_t num_blocks, int32_t dtype, void* plan,
                                           int64_t plan_bytes, void* stream) {
  using namespace nkv;
  if (int rc = check_sg_geometry("nkv_build_store_gather_plan", num_tokens, num_seqs, out_rows,
                                 block_size, row_elems, num_blocks, dtype)) {
    return rc;
  }
  if (table_stride < 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_store_gather_plan: negative table_stride");
  }
  const int64_t need = nkv_store_gather_plan_bytes(num_tokens, out_rows, num_seqs, block_size,
                                                   row_elems, dtype);
  if (int rc = check_plan_bytes("nkv_build_store_gather_plan", plan_bytes, need)) return rc;
  if (need == 0) return NKV_OK;
  if (!plan || (num_seqs > 0 && (!cu_seqlens_q || !cu_seqlens_k)) ||
      (num_seqs > 0 && table_stride > 0 && !block_tables)) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_store_gather_plan: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_store_gather_plan: plan must be 16-byte aligned");
  }
  const int64_t capacity = (need - meta_bytes(num_tokens)) / 16;
  const int64_t chunk_rows = nkv_gather_plan_rows(block_size, row_elems, dtype);
  auto* base = static_cast<uint8_t*>(plan);
  const int64_t items = capacity > num_tokens ? capacity : num_tokens;
  int64_t blocks = (items + kSgPlanThreads - 1) / kSgPlanThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
  const size_t lds = (static_cast<size_t>(num_seqs) + 1 + kSgPlanThreads / kWave + 1) *
                     sizeof(int32_t);
  store_gather_plan_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kSgPlanThreads), lds,
                             static_cast<hipStream_t>(stream)>>>(
      block_tables, table_stride, cu_seqlens_q, cu_seqlens_k, static_cast<int32_t>(num_seqs),
      static_cast<int32_t>(num_tokens), static_cast<int32_t>(block_size),
      static_cast<int32_t>(chunk_rows), num_blocks, out_rows, reinterpret_cast<int2*>(base),
      reinterpret_cast<int4*>(base + meta_bytes(num_tokens)), capacity);
  return nkv_check_launch("nkv_build_store_gather_plan");
}

extern "C" int nkv_store_gather(const void* key, const void* value, void* key_cache,
                                void* value_cache, const int32_t* slot_mapping,
                                int64_t num_tokens, int64_t key_token_stride,
                                int64_t value_token_stride, const void* plan,
                                int64_t plan_bytes, int64_t num_seqs, int64_t out_rows,
                                int64_t block_size, int64_t row_elems, int64_t num_blocks,
                                int32_t dtype, void* key_out, void* value_out, void* stream) {
  using namespace nkv;
  if (int rc = check_sg_geometry("nkv_store_gather", num_tokens, num_seqs, out_rows, block_size,
                                 row_elems, num_blocks, dtype)) {
    return rc;
  }
  if (key_token_stride < 0 || value_token_stride < 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_store_gather: negative token stride");
  }
  const int64_t need = nkv_store_gather_plan_bytes(num_tokens, out_rows, num_seqs, block_size,
                                                   row_elems, dtype);
  if (int rc = check_plan_bytes("nkv_store_gather", plan_bytes, need)) return rc;
  if (num_tokens == 0 && out_rows == 0) return NKV_OK;
  if (!key_cache || !value_cache || !plan || (num_tokens > 0 && (!key || !value || !slot_mapping)) ||
      (out_rows > 0 && (!key_out || !value_out))) {
    return nkv_fail(NKV_E_INVALID, "nkv_store_gather: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_store_gather: plan must be 16-byte aligned");
  }
  const int eb = element_bytes(dtype);
  const int64_t row_bytes = row_elems * eb;
  const int64_t ks = key_token_stride * eb;
  const int64_t vs = value_token_stride * eb;
  const int64_t capacity = (need - meta_bytes(num_tokens)) / 16;
  const int64_t chunk_rows = nkv_gather_plan_rows(block_size, row_elems, dtype);
  const int w = common_word_bytes(
      {reinterpret_cast<uint64_t>(key), reinterpret_cast<uint64_t>(value),
       reinterpret_cast<uint64_t>(key_cache), reinterpret_cast<uint64_t>(value_cache),
       reinterpret_cast<uint64_t>(key_out), reinterpret_cast<uint64_t>(value_out),
       static_cast<uint64_t>(ks), static_cast<uint64_t>(vs), static_cast<uint64_t>(row_bytes)});
  if (row_bytes / w > INT32_MAX) return nkv_fail(NKV_E_INVALID, "nkv_store_gather: row too large");
  const auto* base = static_cast<const uint8_t*>(plan);
  const auto* meta = reinterpret_cast<const int2*>(base);
  const auto* entries = reinterpret_cast<const int4*>(base + meta_bytes(num_tokens));
  const int64_t num_slots = num_blocks * block_size;
  const auto n = static_cast<int32_t>(num_tokens);
  hipStream_t s = static_cast<hipStream_t>(stream);
#define NKV_SG(WB)                                                                           \
  return launch_store_gather<WB>(key, value, key_cache, value_cache, slot_mapping, meta, n, ks, \
                                 vs, row_bytes, num_slots, entries, capacity, chunk_rows,    \
                                 out_rows, key_out, value_out, s)
  switch (w) {
    case 16:
      NKV_SG(16);
    case 8:
      NKV_SG(8);
    case 4:
      NKV_SG(4);
    case 2:
      NKV_SG(2);
    default:
      return nkv_fail(NKV_E_INVALID,
                      "nkv_store_gather: pointers/strides not aligned to the element size");
  }
#undef NKV_SG
}
