// Paged KV gather: build contiguous K/V from the paged caches.
//
// The rows of one cache block are contiguous in memory (block_size rows of
// row_bytes each), so a sequence's context is a list of contiguous runs, one
// per logical block.  The copies are HBM-bound streaming moves: 16-byte
// words, consecutive lanes on consecutive words, non-temporal loads and
// stores, no LDS staging of payload and no MFMA.
//
// Launch shape (measured on MI355X, decode-step gather of 7.3 GB): many
// short-lived 128-thread workgroups, each moving ~4 KiB of ONE tensor with
// a single load in flight per lane (load, store, load, store), reach
// ~6.4 TB/s; long-lived workgroups streaming 32 KiB with 8 loads in flight
// per lane stay near 5.3 TB/s, two loads in flight per lane lose ~10%, and
// a workgroup that moves K and V together (four concurrent streams) loses
// to K and V in separate workgroups.  The write side is the limit: on this
// part pure writes top out near 5.6 TB/s while pure non-temporal reads
// reach 7.2 TB/s.  So the gather launches one workgroup per "sub-chunk" of
// sub_rows rows (sub_rows * row_bytes <= NKV_GATHER_WG_BYTES), with
// blockIdx.y selecting K or V; all K workgroups dispatch before the V ones.
//
//  * gather_seq_kernel   — the reference op gather(cache, table, L)
//    (csrc/paged_kv/paged_kv_cuda.cu:61-94,134-164; oracle
//    nanovllm/layers/paged_kv/pytorch_backend.py:40-50); each workgroup reads
//    its source block straight from the table.
//  * build_plan_kernel   — turns block_tables + cu_seqlens_k of a whole batch
//    into a flat list of chunks {src_row, dst_row, num_rows, seq} of
//    chunk_rows rows (a divisor of block_size); every workgroup rescans the
//    per-sequence chunk counts in LDS (wavefront prefix scan), so the plan
//    needs one launch and no grid-wide sync.
//  * gather_planned_kernel — one launch gathers K and V of every sequence of
//    the batch from a plan (chunk_rows / sub_rows workgroups per entry),
//    replacing the reference's per-request loop
//    (nanovllm/layers/attention.py:250-259, 284-292) of one launch per
//    (request, K or V).
#include <cstdlib>

#include "nkv_common.h"

namespace nkv {
namespace {

// Launch-shape knobs (compile-time, for tuning sweeps): workgroup size,
// words in flight per lane per tensor, whether payload loads / stores carry
// the non-temporal hint, the plan granularity, the bytes one workgroup
// moves, and whether K and V go to separate workgroups.
#ifndef NKV_GATHER_THREADS
#define NKV_GATHER_THREADS 128
#endif
#ifndef NKV_GATHER_UNROLL
#define NKV_GATHER_UNROLL 1
#endif
#ifndef NKV_GATHER_WG_BYTES
#define NKV_GATHER_WG_BYTES 4096
#endif
#ifndef NKV_GATHER_SPLIT_KV
#define NKV_GATHER_SPLIT_KV 1
#endif
#ifndef NKV_GATHER_NT_LOADS
#define NKV_GATHER_NT_LOADS 1
#endif
#ifndef NKV_GATHER_NT_STORES
#define NKV_GATHER_NT_STORES 1
#endif
#ifndef NKV_GATHER_CHUNK_BYTES
#define NKV_GATHER_CHUNK_BYTES 32768
#endif

constexpr int kGatherThreads = NKV_GATHER_THREADS;
constexpr int kGatherUnroll = NKV_GATHER_UNROLL;
constexpr int kPlanThreads = 1024;
constexpr int64_t kDefaultChunkBytes = NKV_GATHER_CHUNK_BYTES;

template <typename T>
__device__ __forceinline__ T load_payload(const T* p) {
  if constexpr (NKV_GATHER_NT_LOADS) return load_stream(p);
  return *p;
}
template <typename T>
__device__ __forceinline__ void store_payload(T* p, T v) {
  if constexpr (NKV_GATHER_NT_STORES) {
    store_stream(p, v);
  } else {
    *p = v;
  }
}

int64_t chunk_bytes_target() {
  static const int64_t value = [] {
    const char* env = std::getenv("NKV_GATHER_CHUNK_BYTES");
    if (env != nullptr) {
      const long long v = std::atoll(env);
      if (v >= 16 && v <= (int64_t{1} << 30)) return static_cast<int64_t>(v);
    }
    return kDefaultChunkBytes;
  }();
  return value;
}

// Largest divisor of `rows` that is <= max(1, target_bytes / row_bytes).
int64_t divisor_rows(int64_t rows, int64_t row_bytes, int64_t target_bytes) {
  int64_t target = target_bytes / row_bytes;
  if (target < 1) target = 1;
  if (target >= rows) return rows;
  for (int64_t r = target; r > 1; --r) {
    if (rows % r == 0) return r;
  }
  return 1;
}

// Plan granularity: a divisor of block_size, ~NKV_GATHER_CHUNK_BYTES.
int64_t chunk_rows_for(int64_t block_size, int64_t row_bytes) {
  return divisor_rows(block_size, row_bytes, chunk_bytes_target());
}

// Rows one workgroup moves: a divisor of `rows` (the plan chunk, or the
// block for the single-sequence gather), ~NKV_GATHER_WG_BYTES.
int64_t sub_rows_for(int64_t rows, int64_t row_bytes) {
  return divisor_rows(rows, row_bytes, NKV_GATHER_WG_BYTES);
}

// Copies nwords words from s0 to d0 (and s1 to d1 when TWO) with the whole
// workgroup: kGatherUnroll loads per tensor in flight per lane, consecutive
// lanes on consecutive words (a wavefront covers 64 x W bytes per access).
template <int W, bool TWO>
__device__ __forceinline__ void copy_chunk(const uint8_t* __restrict__ src0,
                                           uint8_t* __restrict__ dst0,
                                           const uint8_t* __restrict__ src1,
                                           uint8_t* __restrict__ dst1,
                                           int32_t nwords) {
  using T = typename Word<W>::type;
  const T* s0 = reinterpret_cast<const T*>(src0);
  const T* s1 = reinterpret_cast<const T*>(src1);
  T* d0 = reinterpret_cast<T*>(dst0);
  T* d1 = reinterpret_cast<T*>(dst1);
  constexpr int32_t kStep = kGatherThreads * kGatherUnroll;
  int32_t i = threadIdx.x;
  for (; i + (kGatherUnroll - 1) * kGatherThreads < nwords; i += kStep) {
    T a[kGatherUnroll];
    T b[kGatherUnroll];
#pragma unroll
    for (int u = 0; u < kGatherUnroll; ++u) {
      a[u] = load_payload(s0 + i + u * kGatherThreads);
      if constexpr (TWO) b[u] = load_payload(s1 + i + u * kGatherThreads);
    }
#pragma unroll
    for (int u = 0; u < kGatherUnroll; ++u) {
      store_payload(d0 + i + u * kGatherThreads, a[u]);
      if constexpr (TWO) store_payload(d1 + i + u * kGatherThreads, b[u]);
    }
  }
  for (; i < nwords; i += kGatherThreads) {
    const T a = load_payload(s0 + i);
    T b{};
    if constexpr (TWO) b = load_payload(s1 + i);
    store_payload(d0 + i, a);
    if constexpr (TWO) store_payload(d1 + i, b);
  }
}

template <int W, bool TWO>
__device__ __forceinline__ void zero_chunk(uint8_t* __restrict__ dst0,
                                           uint8_t* __restrict__ dst1,
                                           int32_t nwords) {
  using T = typename Word<W>::type;
  T* d0 = reinterpret_cast<T*>(dst0);
  T* d1 = reinterpret_cast<T*>(dst1);
  for (int32_t i = threadIdx.x; i < nwords; i += kGatherThreads) {
    d0[i] = T{};
    if constexpr (TWO) d1[i] = T{};
  }
}

template <int W>
__global__ __launch_bounds__(kGatherThreads) void gather_seq_kernel(
    const uint8_t* __restrict__ cache, const int32_t* __restrict__ table,
    int32_t seq_len, int32_t block_size, int32_t chunk_rows,
    int64_t row_bytes, int64_t num_blocks, uint8_t* __restrict__ out) {
  const int32_t row0 = blockIdx.x * chunk_rows;  // < seq_len by the grid
  const int32_t nrows = min(chunk_rows, seq_len - row0);
  const int32_t block = table[row0 / block_size];
  uint8_t* dst = out + row0 * row_bytes;
  const auto nwords = static_cast<int32_t>(nrows * row_bytes / W);
  if (block < 0 || block >= num_blocks) {
    zero_chunk<W, false>(dst, nullptr, nwords);
    return;
  }
  const int64_t src_row =
      static_cast<int64_t>(block) * block_size + row0 % block_size;
  copy_chunk<W, false>(cache + src_row * row_bytes, dst, nullptr, nullptr,
                       nwords);
}

// Plan entry layout: x = source row (block*block_size + offset, -1 when the
// block id is invalid), y = destination row, z = rows, w = sequence index.
// first_chunk (optional, [num_seqs + 1]) receives the index of every
// sequence's first entry, i.e. the exclusive scan of the chunk counts.
__global__ __launch_bounds__(kPlanThreads) void build_plan_kernel(
    const int32_t* __restrict__ tables, int64_t table_stride,
    const int32_t* __restrict__ cu_seqlens, int32_t num_seqs,
    int32_t block_size, int32_t chunk_rows, int64_t num_blocks,
    int64_t out_rows, int4* __restrict__ plan, int64_t capacity,
    int32_t* __restrict__ first_chunk) {
  extern __shared__ int32_t s_mem[];
  int32_t* s_first = s_mem;                 // [num_seqs + 1]
  int32_t* s_tmp = s_mem + num_seqs + 1;    // [kPlanThreads / 64 + 1]
  lds_exclusive_scan<kPlanThreads>(
      num_seqs,
      [&](int32_t i) {
        const int32_t len = cu_seqlens[i + 1] - cu_seqlens[i];
        return len > 0 ? (len + chunk_rows - 1) / chunk_rows : 0;
      },
      s_first, s_tmp);
  if (first_chunk != nullptr && blockIdx.x == 0) {
    for (int32_t i = threadIdx.x; i <= num_seqs; i += kPlanThreads) first_chunk[i] = s_first[i];
  }
  const int64_t total = s_first[num_seqs];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kPlanThreads;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kPlanThreads + threadIdx.x;
       e < capacity; e += stride) {
    int4 entry = make_int4(0, 0, 0, 0);
    if (e < total) {
      const int32_t i = owner_of(s_first, num_seqs, static_cast<int32_t>(e));
      const int32_t row0 = (static_cast<int32_t>(e) - s_first[i]) * chunk_rows;
      const int32_t base = cu_seqlens[i];
      const int32_t len = cu_seqlens[i + 1] - base;
      int64_t nrows = min(chunk_rows, len - row0);
      const int64_t dst = static_cast<int64_t>(base) + row0;
      // Never write outside the caller's [out_rows] output.
      if (dst < 0 || dst >= out_rows) nrows = 0;
      if (dst + nrows > out_rows) nrows = out_rows - dst;
      const int64_t logical = row0 / block_size;
      int32_t src = -1;
      if (logical < table_stride) {
        const int32_t block = tables[i * table_stride + logical];
        if (block >= 0 && block < num_blocks) {
          src = block * block_size + row0 % block_size;
        }
      }
      entry = make_int4(src, static_cast<int32_t>(dst),
                        static_cast<int32_t>(nrows), i);
    }
    plan[e] = entry;
  }
}

// One workgroup per sub-chunk of a plan entry: blockIdx.x = entry *
// subs_per_entry + sub, blockIdx.y = 0 for K, 1 for V (or one workgroup
// moving both when SPLIT is false).  Plan entries are re-checked against the
// actual cache and output sizes (workgroup-uniform scalar compares), so a
// plan built for another geometry can never make this kernel read or write
// out of bounds.
template <int W, bool TWO_IN_ONE>
__global__ __launch_bounds__(kGatherThreads) void gather_planned_kernel(
    const uint8_t* __restrict__ key_cache,
    const uint8_t* __restrict__ value_cache, const int4* __restrict__ plan,
    int32_t subs_per_entry, int32_t sub_rows, int64_t cache_rows,
    int64_t out_rows, int64_t row_bytes, uint8_t* __restrict__ key_out,
    uint8_t* __restrict__ value_out) {
  const int32_t e = blockIdx.x / subs_per_entry;
  const int32_t row_off = (blockIdx.x - e * subs_per_entry) * sub_rows;
  const int4 entry = plan[e];
  if (entry.z <= row_off || entry.y < 0 ||
      static_cast<int64_t>(entry.y) + entry.z > out_rows) {
    return;
  }
  const int32_t nrows = min(sub_rows, entry.z - row_off);
  const bool second = blockIdx.y != 0;
  const uint8_t* cache = second ? value_cache : key_cache;
  uint8_t* out = second ? value_out : key_out;
  const int64_t dst = (static_cast<int64_t>(entry.y) + row_off) * row_bytes;
  const auto nwords = static_cast<int32_t>(nrows * row_bytes / W);
  if (entry.x < 0 || static_cast<int64_t>(entry.x) + entry.z > cache_rows) {
    zero_chunk<W, TWO_IN_ONE>(out + dst, value_out + dst, nwords);
    return;
  }
  const int64_t src = (static_cast<int64_t>(entry.x) + row_off) * row_bytes;
  copy_chunk<W, TWO_IN_ONE>(cache + src, out + dst, value_cache + src,
                            value_out + dst, nwords);
}

template <int W>
int launch_gather_seq(const void* cache, const int32_t* table, int32_t len,
                      int64_t block_size, int64_t chunk_rows,
                      int64_t row_bytes, int64_t num_blocks, void* out,
                      hipStream_t stream) {
  const int64_t chunks = (len + chunk_rows - 1) / chunk_rows;
  gather_seq_kernel<W><<<dim3(static_cast<unsigned>(chunks)),
                         dim3(kGatherThreads), 0, stream>>>(
      static_cast<const uint8_t*>(cache), table, len,
      static_cast<int32_t>(block_size), static_cast<int32_t>(chunk_rows),
      row_bytes, num_blocks, static_cast<uint8_t*>(out));
  return nkv_check_launch("nkv_gather");
}

template <int W, bool TWO_IN_ONE>
int launch_planned(const void* key_cache, const void* value_cache,
                   const void* plan, int64_t capacity, int64_t subs,
                   int64_t sub_rows, int64_t cache_rows, int64_t out_rows,
                   int64_t row_bytes, void* key_out, void* value_out,
                   unsigned grid_y, hipStream_t stream) {
  gather_planned_kernel<W, TWO_IN_ONE>
      <<<dim3(static_cast<unsigned>(capacity * subs), grid_y),
         dim3(kGatherThreads), 0, stream>>>(
      static_cast<const uint8_t*>(key_cache),
      static_cast<const uint8_t*>(value_cache),
      static_cast<const int4*>(plan), static_cast<int32_t>(subs),
      static_cast<int32_t>(sub_rows), cache_rows, out_rows, row_bytes,
      static_cast<uint8_t*>(key_out), static_cast<uint8_t*>(value_out));
  return nkv_check_launch("nkv_gather_varlen_planned");
}

int check_geometry(const char* what, int64_t block_size, int64_t row_elems,
                   int64_t num_blocks, int32_t dtype) {
  const int eb = element_bytes(dtype);
  if (eb == 0) return nkv_fail(NKV_E_INVALID, "%s: unknown dtype %d", what, dtype);
  if (block_size <= 0 || row_elems <= 0 || num_blocks < 0) {
    return nkv_fail(NKV_E_INVALID,
                    "%s: block_size and row_elems must be positive, "
                    "num_blocks non-negative",
                    what);
  }
  if (num_blocks * block_size > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID,
                    "%s: num_blocks*block_size exceeds int32 rows", what);
  }
  if (block_size * row_elems * eb > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "%s: cache block exceeds 2 GiB", what);
  }
  return NKV_OK;
}

}  // namespace

// Shared by the gather plan and the decode-attention partition plan
// (chunk_rows = block_size); arguments are validated by the callers.
int launch_block_plan(const int32_t* tables, int64_t table_stride,
                      const int32_t* cu_seqlens, int64_t num_seqs,
                      int64_t out_rows, int64_t block_size, int64_t chunk_rows,
                      int64_t num_blocks, int32_t* plan, int64_t capacity,
                      int32_t* first_chunk, hipStream_t stream,
                      const char* what) {
  int64_t blocks = (capacity + kPlanThreads - 1) / kPlanThreads;
  if (blocks < 1) blocks = 1;
  if (blocks > 1024) blocks = 1024;
  const size_t lds = (static_cast<size_t>(num_seqs) + 1 + kPlanThreads / kWave + 1) *
                     sizeof(int32_t);
  build_plan_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kPlanThreads),
                      lds, stream>>>(
      tables, table_stride, cu_seqlens, static_cast<int32_t>(num_seqs),
      static_cast<int32_t>(block_size), static_cast<int32_t>(chunk_rows), num_blocks,
      out_rows, reinterpret_cast<int4*>(plan), capacity, first_chunk);
  return nkv_check_launch(what);
}

}  // namespace nkv

extern "C" int64_t nkv_gather_plan_rows(int64_t block_size, int64_t row_elems,
                                        int32_t dtype) {
  const int eb = nkv::element_bytes(dtype);
  if (eb == 0 || block_size <= 0 || row_elems <= 0) return 0;
  return nkv::chunk_rows_for(block_size, row_elems * eb);
}

extern "C" int64_t nkv_gather_plan_capacity(int64_t total_rows,
                                            int64_t num_seqs,
                                            int64_t block_size,
                                            int64_t row_elems, int32_t dtype) {
  const int64_t rows = nkv_gather_plan_rows(block_size, row_elems, dtype);
  if (rows <= 0 || total_rows < 0 || num_seqs < 0) return 0;
  return (total_rows + rows - 1) / rows + num_seqs;
}

extern "C" int nkv_gather(const void* cache, const int32_t* block_table,
                          int64_t table_len, int64_t sequence_length,
                          int64_t block_size, int64_t row_elems,
                          int64_t num_blocks, int32_t dtype, void* out,
                          void* stream) {
  using namespace nkv;
  if (int rc = check_geometry("nkv_gather", block_size, row_elems, num_blocks, dtype)) {
    return rc;
  }
  if (sequence_length < 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather: sequence_length must be non-negative");
  }
  if (sequence_length == 0) return NKV_OK;
  if (sequence_length > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather: sequence_length exceeds int32");
  }
  const int64_t required = (sequence_length + block_size - 1) / block_size;
  if (table_len < required) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_gather: block_table does not cover the requested "
                    "sequence length (%lld < %lld blocks)",
                    static_cast<long long>(table_len),
                    static_cast<long long>(required));
  }
  if (!cache || !block_table || !out) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather: null pointer");
  }
  const int64_t row_bytes = row_elems * element_bytes(dtype);
  const int64_t rows = sub_rows_for(block_size, row_bytes);
  const int w = common_word_bytes({reinterpret_cast<uint64_t>(cache),
                                   reinterpret_cast<uint64_t>(out),
                                   static_cast<uint64_t>(row_bytes)});
  const auto len = static_cast<int32_t>(sequence_length);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (w) {
    case 16:
      return launch_gather_seq<16>(cache, block_table, len, block_size, rows, row_bytes, num_blocks, out, s);
    case 8:
      return launch_gather_seq<8>(cache, block_table, len, block_size, rows, row_bytes, num_blocks, out, s);
    case 4:
      return launch_gather_seq<4>(cache, block_table, len, block_size, rows, row_bytes, num_blocks, out, s);
    case 2:
      return launch_gather_seq<2>(cache, block_table, len, block_size, rows, row_bytes, num_blocks, out, s);
    default:
      return nkv_fail(NKV_E_INVALID, "nkv_gather: pointers not aligned to the element size");
  }
}

extern "C" int nkv_build_gather_plan(const int32_t* block_tables,
                                     int64_t table_stride,
                                     const int32_t* cu_seqlens_k,
                                     int64_t num_seqs, int64_t out_rows,
                                     int64_t block_size, int64_t row_elems,
                                     int64_t num_blocks, int32_t dtype,
                                     void* plan, int64_t capacity,
                                     void* stream) {
  using namespace nkv;
  if (int rc = check_geometry("nkv_build_gather_plan", block_size, row_elems, num_blocks, dtype)) {
    return rc;
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_build_gather_plan: num_seqs=%lld outside [0, %d]",
                    static_cast<long long>(num_seqs), NKV_MAX_PLAN_SEQS);
  }
  if (capacity < 0 || capacity > INT32_MAX || out_rows < 0 || out_rows > INT32_MAX ||
      table_stride < 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_build_gather_plan: capacity/out_rows/table_stride "
                    "out of range");
  }
  if (capacity == 0) return NKV_OK;
  if (!plan || (num_seqs > 0 && (!block_tables || !cu_seqlens_k))) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_gather_plan: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_gather_plan: plan must be 16-byte aligned");
  }
  const int64_t row_bytes = row_elems * element_bytes(dtype);
  const int64_t rows = chunk_rows_for(block_size, row_bytes);
  return launch_block_plan(block_tables, table_stride, cu_seqlens_k, num_seqs,
                           out_rows, block_size, rows, num_blocks,
                           static_cast<int32_t*>(plan), capacity, nullptr,
                           static_cast<hipStream_t>(stream),
                           "nkv_build_gather_plan");
}

extern "C" int nkv_gather_varlen_planned(const void* key_cache,
                                         const void* value_cache,
                                         const void* plan, int64_t capacity,
                                         int64_t cache_rows, int64_t out_rows,
                                         int64_t block_size, int64_t row_elems,
                                         int32_t dtype,
                                         void* key_out, void* value_out,
                                         void* stream) {
  using namespace nkv;
  const int eb = element_bytes(dtype);
  if (eb == 0) return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_planned: unknown dtype %d", dtype);
  if (row_elems <= 0 || capacity < 0 || capacity > INT32_MAX || cache_rows < 0 ||
      out_rows < 0 || cache_rows > INT32_MAX || out_rows > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_gather_varlen_planned: bad row_elems/capacity/cache_rows/out_rows");
  }
  if (capacity == 0 || out_rows == 0) return NKV_OK;
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_planned: plan must be 16-byte aligned");
  }
  const bool two = value_cache != nullptr;
  if (!key_cache || !key_out || !plan || (two != (value_out != nullptr))) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_gather_varlen_planned: null pointer (value_cache and "
                    "value_out must be both set or both NULL)");
  }
  const int64_t row_bytes = row_elems * eb;
  if (block_size <= 0 || block_size > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_planned: block_size must be positive");
  }
  const int64_t chunk_rows = chunk_rows_for(block_size, row_bytes);
  const int64_t sub_rows = sub_rows_for(chunk_rows, row_bytes);
  const int64_t subs = chunk_rows / sub_rows;
  if (capacity * subs > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen_planned: plan too large for one launch");
  }
  const int w = common_word_bytes(
      {reinterpret_cast<uint64_t>(key_cache), reinterpret_cast<uint64_t>(key_out),
       reinterpret_cast<uint64_t>(two ? value_cache : key_cache),
       reinterpret_cast<uint64_t>(two ? value_out : key_out),
       static_cast<uint64_t>(row_bytes)});
  hipStream_t s = static_cast<hipStream_t>(stream);
  // K and V in separate workgroups (grid y = 2) unless NKV_GATHER_SPLIT_KV=0.
  const bool together = two && !NKV_GATHER_SPLIT_KV;
  const unsigned grid_y = (two && NKV_GATHER_SPLIT_KV) ? 2u : 1u;
#define NKV_PLANNED(WB)                                                        \
  return together ? launch_planned<WB, true>(key_cache, value_cache, plan,    \
                                             capacity, subs, sub_rows,        \
                                             cache_rows, out_rows, row_bytes, \
                                             key_out, value_out, 1u, s)       \
                  : launch_planned<WB, false>(key_cache, value_cache, plan,   \
                                              capacity, subs, sub_rows,       \
                                              cache_rows, out_rows, row_bytes,\
                                              key_out, value_out, grid_y, s)
  switch (w) {
    case 16:
      NKV_PLANNED(16);
    case 8:
      NKV_PLANNED(8);
    case 4:
      NKV_PLANNED(4);
    case 2:
      NKV_PLANNED(2);
    default:
      return nkv_fail(NKV_E_INVALID,
                      "nkv_gather_varlen_planned: pointers not aligned to the "
                      "element size");
  }
#undef NKV_PLANNED
}

extern "C" int nkv_gather_varlen(const void* key_cache, const void* value_cache,
                                 const int32_t* block_tables,
                                 int64_t table_stride,
                                 const int32_t* cu_seqlens_k, int64_t num_seqs,
                                 int64_t total_rows, int64_t block_size,
                                 int64_t row_elems, int64_t num_blocks,
                                 int32_t dtype, void* key_out, void* value_out,
                                 void* workspace, int64_t workspace_bytes,
                                 void* stream) {
  const int64_t capacity =
      nkv_gather_plan_capacity(total_rows, num_seqs, block_size, row_elems, dtype);
  if (total_rows == 0) return NKV_OK;
  if (capacity <= 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_gather_varlen: bad geometry");
  }
  if (workspace_bytes < capacity * 16) {
    return nkv_fail(NKV_E_CAPACITY,
                    "nkv_gather_varlen: workspace of %lld bytes < %lld needed",
                    static_cast<long long>(workspace_bytes),
                    static_cast<long long>(capacity * 16));
  }
  if (int rc = nkv_build_gather_plan(block_tables, table_stride, cu_seqlens_k,
                                     num_seqs, total_rows, block_size,
                                     row_elems, num_blocks, dtype, workspace,
                                     capacity, stream)) {
    return rc;
  }
  return nkv_gather_varlen_planned(key_cache, value_cache, workspace, capacity,
                                   num_blocks * block_size, total_rows,
                                   block_size, row_elems, dtype, key_out,
                                   value_out, stream);
}
