// Shared device helpers for the nanokv paged-KV kernels (gfx950 / CDNA4).
//
// Everything here moves bytes: K/V rows are copied as opaque 2-, 4-, 8- or
// 16-byte words, never converted, so results are bit-identical to the source
// for every dtype.  Wavefronts are 64 lanes wide; the widest word is 16 bytes
// (global_load_dwordx4 / global_store_dwordx4), so one wavefront moves 1 KiB
// per instruction.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <initializer_list>

#include "nanokv.h"

namespace nkv {

constexpr int kWave = 64;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

template <int BYTES>
struct Word;
template <>
struct Word<16> {
  using type = u32x4;
};
template <>
struct Word<8> {
  using type = u32x2;
};
template <>
struct Word<4> {
  using type = uint32_t;
};
template <>
struct Word<2> {
  using type = uint16_t;
};

// Streaming (non-temporal) accesses: the gathered rows are read once from
// the cache and written once to the output, so neither side should displace
// useful lines from L2 / MALL.
template <typename T>
__device__ __forceinline__ T load_stream(const T* p) {
  return __builtin_nontemporal_load(p);
}
template <typename T>
__device__ __forceinline__ void store_stream(T* p, T v) {
  __builtin_nontemporal_store(v, p);
}

// Largest power of two <= 16 that divides every value (byte addresses,
// byte strides, byte row sizes).  It picks the widest word every access of
// a launch can use with natural alignment.
inline int common_word_bytes(std::initializer_list<uint64_t> values) {
  int w = 16;
  for (uint64_t v : values) {
    while (w > 1 && (v % static_cast<uint64_t>(w)) != 0) w >>= 1;
  }
  return w;
}

// Inclusive scan of one int32 per lane across a 64-lane wavefront
// (log2(64) = 6 shuffle steps).
__device__ __forceinline__ int32_t wave_inclusive_scan(int32_t x) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    const int32_t y = __shfl_up(x, d, kWave);
    if (lane >= d) x += y;
  }
  return x;
}

__device__ __forceinline__ int32_t wave_max(int32_t x) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) x = max(x, __shfl_xor(x, d, kWave));
  return x;
}

// Exclusive scan of one value per thread across a workgroup of NT threads:
// wavefront scans, then one wavefront scans the per-wave totals held in
// LDS.  s_tmp needs NT/64 + 1 ints.  Returns the thread's exclusive prefix
// and writes the workgroup total to *total.  Must be reached by every
// thread of the workgroup.
template <int NT>
__device__ __forceinline__ int32_t block_exclusive_scan(int32_t v,
                                                        int32_t* s_tmp,
                                                        int32_t* total) {
  static_assert(NT % kWave == 0 && NT / kWave <= kWave, "bad workgroup size");
  constexpr int kWaves = NT / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int wid = threadIdx.x / kWave;
  const int32_t incl = wave_inclusive_scan(v);
  if (lane == kWave - 1) s_tmp[wid] = incl;
  __syncthreads();
  if (wid == 0) {
    const int32_t w = lane < kWaves ? s_tmp[lane] : 0;
    const int32_t wi = wave_inclusive_scan(w);
    if (lane < kWaves) s_tmp[lane] = wi - w;
    if (lane == kWaves - 1) s_tmp[kWaves] = wi;
  }
  __syncthreads();
  const int32_t result = s_tmp[wid] + incl - v;
  *total = s_tmp[kWaves];
  __syncthreads();  // s_tmp may be reused by the caller afterwards
  return result;
}

// Exclusive scan of f(i), i in [0, n), into s_out[0..n] (s_out[n] = total),
// each thread handling a run of consecutive items.  s_out needs n+1 ints of
// LDS, s_tmp NT/64+1.  Ends with a barrier, so s_out is readable by all.
template <int NT, typename F>
__device__ __forceinline__ void lds_exclusive_scan(int32_t n, F f,
                                                   int32_t* s_out,
                                                   int32_t* s_tmp) {
  const int32_t per = (n + NT - 1) / NT;
  const int32_t begin = min(n, static_cast<int32_t>(threadIdx.x) * per);
  const int32_t end = min(n, begin + per);
  int32_t sum = 0;
  for (int32_t i = begin; i < end; ++i) {
    const int32_t v = f(i);
    s_out[i] = v;
    sum += v;
  }
  int32_t total = 0;
  int32_t base = block_exclusive_scan<NT>(sum, s_tmp, &total);
  for (int32_t i = begin; i < end; ++i) {
    const int32_t v = s_out[i];
    s_out[i] = base;
    base += v;
  }
  if (threadIdx.x == 0) s_out[n] = total;
  __syncthreads();
}

// Largest i in [0, n) with s[i] <= key, for s non-decreasing with
// s[0] <= key < s[n]: the owner of item `key` in an exclusive scan.
__device__ __forceinline__ int32_t owner_of(const int32_t* s, int32_t n,
                                            int32_t key) {
  int32_t lo = 0, hi = n;
  while (hi - lo > 1) {
    const int32_t mid = (lo + hi) >> 1;
    if (s[mid] <= key)
      lo = mid;
    else
      hi = mid;
  }
  return lo;
}

// Element size of an NKV_DTYPE_* code, 0 for an unknown code
// (defined in nkv_api.hip).
int element_bytes(int32_t dtype);

// Launches the block-table plan builder (defined in nkv_gather.hip): one
// int4 entry {src_row (-1 if the block id is invalid), dst_row, rows, seq}
// per chunk of chunk_rows rows (a divisor of block_size) of every sequence
// in cu_seqlens; first_chunk (optional, [num_seqs+1]) gets each sequence's
// first entry index.  Callers validate the arguments.
int launch_block_plan(const int32_t* tables, int64_t table_stride,
                      const int32_t* cu_seqlens, int64_t num_seqs,
                      int64_t out_rows, int64_t block_size, int64_t chunk_rows,
                      int64_t num_blocks, int32_t* plan, int64_t capacity,
                      int32_t* first_chunk, hipStream_t stream,
                      const char* what);

// Validates a block-pool descriptor and returns the device addresses of its
// block tables [max_seqs, max_blocks_per_seq] and counts [max_seqs]
// (defined in nkv_pool.hip).
int pool_tables(const nkv_pool_desc* pool, const char* what, const int32_t** tables,
                const int32_t** nblk);

}  // namespace nkv

// Error reporting shared by all translation units (defined in nkv_api.hip).
int nkv_fail(int code, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));
int nkv_check_launch(const char* what);
