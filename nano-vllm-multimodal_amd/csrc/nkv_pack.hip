// Ragged-batch metadata packing on the device.
//
// The scheduler's per-sequence state arrives as a few small int32 arrays in
// CSR form (counts per sequence + the concatenated block lists), and the
// kernels expand it into what the store/gather kernels and the attention
// call consume: cu_seqlens, slot_mapping, -1 padded block_tables, context
// lengths.  This replaces the per-sequence / per-token Python loops of
// ModelRunner.prepare_decode / prepare_prefill / prepare_block_tables
// (nanovllm/engine/model_runner.py:696-707, 757-820, 892-938) and their
// separate host-to-device copies.
//
// Every workgroup that needs a prefix over the sequences recomputes it in
// LDS (a wavefront-level scan of at most NKV_MAX_PACK_SEQS values), so one
// launch does the whole expansion without a grid-wide barrier.  Block-table
// rows are written one wavefront per sequence (64 columns per store).
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kPackThreads = 256;
constexpr int kPackWaves = kPackThreads / kWave;
constexpr int kPackMaxBlocks = 1024;

__device__ __forceinline__ int32_t csr_read(const int32_t* __restrict__ ids,
                                            int64_t nnz, int64_t k) {
  return (k >= 0 && k < nnz) ? ids[k] : -1;
}

// Where sequence i's block list comes from.
//   CsrRows:  the host-built CSR (counts per sequence + concatenated ids);
//   PoolRows: the block tables of a device block pool (nkv_pool), row
//             seq_slots[i]; a slot outside the pool reads as an empty list.
struct CsrRows {
  const int32_t* offsets;
  const int32_t* ids;
  int64_t nnz;
  __device__ __forceinline__ int32_t count(int32_t i) const { return offsets[i + 1] - offsets[i]; }
  __device__ __forceinline__ int32_t id(int32_t i, int32_t j) const {
    return csr_read(ids, nnz, static_cast<int64_t>(offsets[i]) + j);
  }
};

struct PoolRows {
  const int32_t* seq_slots;
  const int32_t* tables;
  const int32_t* nblk;
  int32_t max_seqs;
  int32_t width;
  __device__ __forceinline__ int32_t slot(int32_t i) const {
    const int32_t s = seq_slots[i];
    return (s >= 0 && s < max_seqs) ? s : -1;
  }
  __device__ __forceinline__ int32_t count(int32_t i) const {
    const int32_t s = slot(i);
    return s < 0 ? 0 : min(max(nblk[s], 0), width);
  }
  __device__ __forceinline__ int32_t id(int32_t i, int32_t j) const {
    const int32_t s = slot(i);
    return (s < 0 || j < 0 || j >= width) ? -1 : tables[static_cast<int64_t>(s) * width + j];
  }
};

// One wavefront writes block_tables[i, 0:width) for sequence i (rows are
// `stride` entries apart; columns >= width are left as they are).
template <typename Rows>
__device__ __forceinline__ void write_table_row(const Rows& rows, int32_t i, int32_t width,
                                                int64_t stride, int32_t* __restrict__ tables) {
  const int32_t lane = threadIdx.x & (kWave - 1);
  const int32_t count = rows.count(i);
  int32_t* row = tables + static_cast<int64_t>(i) * stride;
  for (int32_t j = lane; j < width; j += kWave) {
    row[j] = j < count ? rows.id(i, j) : -1;
  }
}

// Sequences [num_seqs, padded_seqs) are graph-bucket padding: slot -1,
// context length 0, cu_seqlens_k flat at the total, block-table rows left
// as they are (the fill of model_runner.py:998-1011).
template <typename Rows>
__global__ __launch_bounds__(kPackThreads) void pack_decode_kernel(
    const int32_t* __restrict__ num_tokens, Rows rows, int32_t num_seqs,
    int32_t padded_seqs, int32_t block_size, int32_t width,
    int64_t table_stride, int32_t* __restrict__ slot_mapping,
    int32_t* __restrict__ context_lens, int32_t* __restrict__ tables,
    int32_t* __restrict__ cu_seqlens_k) {
  extern __shared__ int32_t s_mem[];
  if (cu_seqlens_k != nullptr && blockIdx.x == 0) {
    int32_t* s_cu = s_mem;
    int32_t* s_tmp = s_mem + num_seqs + 1;
    lds_exclusive_scan<kPackThreads>(
        num_seqs, [&](int32_t i) { return max(num_tokens[i], 0); }, s_cu,
        s_tmp);
    for (int32_t i = threadIdx.x; i <= padded_seqs; i += kPackThreads) {
      cu_seqlens_k[i] = s_cu[min(i, num_seqs)];
    }
  }
  const int32_t lane = threadIdx.x & (kWave - 1);
  const int32_t num_waves = gridDim.x * kPackWaves;
  for (int32_t i = blockIdx.x * kPackWaves + threadIdx.x / kWave; i < padded_seqs;
       i += num_waves) {
    if (i >= num_seqs) {
      if (lane == 0) {
        slot_mapping[i] = -1;
        if (context_lens != nullptr) context_lens[i] = 0;
      }
      continue;
    }
    if (tables != nullptr) write_table_row(rows, i, width, table_stride, tables);
    if (lane == 0) {
      const int32_t n = num_tokens[i];
      const int32_t count = rows.count(i);
      int32_t slot = -1;
      // slot = block_table[-1]*BS + last_block_num_tokens - 1 with
      // last_block_num_tokens = n - (ceil(n/BS) - 1)*BS
      // (model_runner.py:916, sequence.py:176-183).
      if (count > 0 && n >= 0) {
        const int32_t last = rows.id(i, count - 1);
        if (last >= 0) {
          const int32_t blocks = (n + block_size - 1) / block_size;
          const int32_t last_tokens = n - (blocks - 1) * block_size;
          slot = last * block_size + last_tokens - 1;
        }
      }
      slot_mapping[i] = slot;
      if (context_lens != nullptr) context_lens[i] = n;
    }
  }
}

template <typename Rows>
__global__ __launch_bounds__(kPackThreads) void pack_prefill_kernel(
    const int32_t* __restrict__ num_cached,
    const int32_t* __restrict__ num_scheduled,
    const int32_t* __restrict__ num_prompt, Rows rows, int32_t num_seqs,
    int32_t block_size, int32_t width, int32_t num_slots,
    int32_t* __restrict__ cu_seqlens_q, int32_t* __restrict__ cu_seqlens_k,
    int32_t* __restrict__ slot_mapping, int32_t* __restrict__ tables,
    int32_t* __restrict__ full_context_lens,
    int32_t* __restrict__ query_start_lens, int32_t* __restrict__ max_seqlens) {
  extern __shared__ int32_t s_mem[];
  int32_t* s_slot0 = s_mem;                     // [num_seqs + 1]
  int32_t* s_aux = s_mem + num_seqs + 1;        // [num_seqs + 1]
  int32_t* s_tmp = s_mem + 2 * (num_seqs + 1);  // [kPackWaves + 1]
  int32_t* s_max = s_tmp + kPackWaves + 1;      // [2 * kPackWaves]

  // First slot_mapping index of each sequence: sequences without a block
  // list (warmup) emit no slots (model_runner.py:789-790).
  lds_exclusive_scan<kPackThreads>(
      num_seqs,
      [&](int32_t i) {
        const bool has_blocks = rows.count(i) > 0;
        return has_blocks ? max(num_scheduled[i], 0) : 0;
      },
      s_slot0, s_tmp);

  if (blockIdx.x == 0) {
    if (cu_seqlens_q != nullptr) {
      lds_exclusive_scan<kPackThreads>(
          num_seqs, [&](int32_t i) { return max(num_scheduled[i], 0); }, s_aux,
          s_tmp);
      for (int32_t i = threadIdx.x; i <= num_seqs; i += kPackThreads) {
        cu_seqlens_q[i] = s_aux[i];
      }
      __syncthreads();
    }
    if (cu_seqlens_k != nullptr) {
      lds_exclusive_scan<kPackThreads>(
          num_seqs,
          [&](int32_t i) { return max(num_cached[i] + num_scheduled[i], 0); },
          s_aux, s_tmp);
      for (int32_t i = threadIdx.x; i <= num_seqs; i += kPackThreads) {
        cu_seqlens_k[i] = s_aux[i];
      }
    }
    if (max_seqlens != nullptr) {
      int32_t max_q = 0, max_k = 0;
      for (int32_t i = threadIdx.x; i < num_seqs; i += kPackThreads) {
        max_q = max(max_q, num_scheduled[i]);
        max_k = max(max_k, num_cached[i] + num_scheduled[i]);
      }
      max_q = wave_max(max_q);
      max_k = wave_max(max_k);
      if ((threadIdx.x & (kWave - 1)) == 0) {
        s_max[threadIdx.x / kWave] = max_q;
        s_max[kPackWaves + threadIdx.x / kWave] = max_k;
      }
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int w = 1; w < kPackWaves; ++w) {
          max_q = max(max_q, s_max[w]);
          max_k = max(max_k, s_max[kPackWaves + w]);
        }
        max_seqlens[0] = max_q;
        max_seqlens[1] = max_k;
      }
    }
  }

  const int64_t threads = static_cast<int64_t>(gridDim.x) * kPackThreads;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kPackThreads + threadIdx.x;
  for (int64_t i = tid; i < num_seqs; i += threads) {
    if (full_context_lens != nullptr) full_context_lens[i] = num_prompt[i];
    if (query_start_lens != nullptr) query_start_lens[i] = num_cached[i];
  }

  if (tables != nullptr) {
    const int32_t num_waves = gridDim.x * kPackWaves;
    for (int32_t i = blockIdx.x * kPackWaves + threadIdx.x / kWave;
         i < num_seqs; i += num_waves) {
      write_table_row(rows, i, width, width, tables);
    }
  }

  // slot of position p of sequence i = bt[p / BS]*BS + p % BS for p in
  // [num_cached, num_cached + num_scheduled) (model_runner.py:792-816).
  const int32_t emitted = s_slot0[num_seqs];
  for (int64_t j = tid; j < num_slots; j += threads) {
    int32_t slot = -1;
    if (j < emitted) {
      const int32_t i = owner_of(s_slot0, num_seqs, static_cast<int32_t>(j));
      const int32_t p = num_cached[i] + static_cast<int32_t>(j) - s_slot0[i];
      const int32_t logical = p / block_size;
      if (p >= 0 && logical < rows.count(i)) {
        const int32_t block = rows.id(i, logical);
        if (block >= 0) slot = block * block_size + p % block_size;
      }
    }
    slot_mapping[j] = slot;
  }
}

int check_pack_args(const char* what, int64_t num_block_ids, int64_t num_seqs,
                    int64_t block_size, int64_t width) {
  if (num_seqs < 0 || num_seqs > NKV_MAX_PACK_SEQS) {
    return nkv_fail(NKV_E_INVALID, "%s: num_seqs=%lld outside [0, %d]", what,
                    static_cast<long long>(num_seqs), NKV_MAX_PACK_SEQS);
  }
  if (block_size <= 0 || block_size > INT32_MAX || width < 0 ||
      width > INT32_MAX || num_block_ids < 0) {
    return nkv_fail(NKV_E_INVALID,
                    "%s: block_size must be positive, table_width and "
                    "num_block_ids non-negative",
                    what);
  }
  return NKV_OK;
}

unsigned pack_grid(int64_t num_seqs, int64_t items) {
  int64_t blocks = (num_seqs + kPackWaves - 1) / kPackWaves;
  const int64_t item_blocks = (items + 4 * kPackThreads - 1) / (4 * kPackThreads);
  if (item_blocks > blocks) blocks = item_blocks;
  if (blocks < 1) blocks = 1;
  if (blocks > kPackMaxBlocks) blocks = kPackMaxBlocks;
  return static_cast<unsigned>(blocks);
}

}  // namespace
}  // namespace nkv

extern "C" int nkv_pack_decode(const int32_t* num_tokens,
                               const int32_t* block_offsets,
                               const int32_t* block_ids, int64_t num_block_ids,
                               int64_t num_seqs, int64_t padded_seqs,
                               int64_t block_size, int64_t table_width,
                               int64_t table_stride, int32_t* slot_mapping,
                               int32_t* context_lens, int32_t* block_tables,
                               int32_t* cu_seqlens_k, void* stream) {
  using namespace nkv;
  if (int rc = check_pack_args("nkv_pack_decode", num_block_ids, num_seqs,
                               block_size, table_width)) {
    return rc;
  }
  if (padded_seqs < num_seqs || padded_seqs > NKV_MAX_PACK_SEQS) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_pack_decode: padded_seqs=%lld must be in [num_seqs, %d]",
                    static_cast<long long>(padded_seqs), NKV_MAX_PACK_SEQS);
  }
  if (table_stride < table_width) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_decode: table_stride < table_width");
  }
  // An empty batch still launches when cu_seqlens_k or padding must be
  // written (a kernel rather than a memset, so the call stays
  // graph-capturable).
  if (padded_seqs == 0 && cu_seqlens_k == nullptr) return NKV_OK;
  if ((padded_seqs > 0 && !slot_mapping) ||
      (num_seqs > 0 && (!num_tokens || !block_offsets || (num_block_ids > 0 && !block_ids)))) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_decode: null pointer");
  }
  const size_t lds = cu_seqlens_k != nullptr
                         ? (static_cast<size_t>(num_seqs) + 1 + kPackWaves + 1) * sizeof(int32_t)
                         : 0;
  pack_decode_kernel<<<dim3(pack_grid(padded_seqs, 0)), dim3(kPackThreads), lds,
                       static_cast<hipStream_t>(stream)>>>(
      num_tokens, CsrRows{block_offsets, block_ids, num_block_ids},
      static_cast<int32_t>(num_seqs), static_cast<int32_t>(padded_seqs),
      static_cast<int32_t>(block_size), static_cast<int32_t>(table_width),
      table_stride, slot_mapping, context_lens, block_tables, cu_seqlens_k);
  return nkv_check_launch("nkv_pack_decode");
}

extern "C" int nkv_pack_prefill(
    const int32_t* num_cached, const int32_t* num_scheduled,
    const int32_t* num_prompt, const int32_t* block_offsets,
    const int32_t* block_ids, int64_t num_block_ids, int64_t num_seqs,
    int64_t block_size, int64_t table_width, int64_t num_slots,
    int32_t* cu_seqlens_q, int32_t* cu_seqlens_k, int32_t* slot_mapping,
    int32_t* block_tables, int32_t* full_context_lens,
    int32_t* query_start_lens, int32_t* max_seqlens, void* stream) {
  using namespace nkv;
  if (int rc = check_pack_args("nkv_pack_prefill", num_block_ids, num_seqs,
                               block_size, table_width)) {
    return rc;
  }
  if (num_slots < 0 || num_slots > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_prefill: num_slots out of range");
  }
  if (!num_cached || !num_scheduled || !block_offsets ||
      (num_block_ids > 0 && !block_ids) || (num_slots > 0 && !slot_mapping) ||
      (full_context_lens && !num_prompt)) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_prefill: null pointer");
  }
  const size_t lds =
      (2 * (static_cast<size_t>(num_seqs) + 1) + 3 * kPackWaves + 1) * sizeof(int32_t);
  pack_prefill_kernel<<<dim3(pack_grid(num_seqs, num_slots)),
                        dim3(kPackThreads), lds,
                        static_cast<hipStream_t>(stream)>>>(
      num_cached, num_scheduled, num_prompt, CsrRows{block_offsets, block_ids, num_block_ids},
      static_cast<int32_t>(num_seqs),
      static_cast<int32_t>(block_size), static_cast<int32_t>(table_width),
      static_cast<int32_t>(num_slots), cu_seqlens_q, cu_seqlens_k,
      slot_mapping, block_tables, full_context_lens, query_start_lens,
      max_seqlens);
  return nkv_check_launch("nkv_pack_prefill");
}

namespace {

// The pool's table arrays as a row source.
int pool_rows(const nkv_pool_desc* pool, const int32_t* seq_slots, const char* what,
              nkv::PoolRows* rows) {
  const int32_t* tables = nullptr;
  const int32_t* nblk = nullptr;
  if (int rc = nkv::pool_tables(pool, what, &tables, &nblk)) return rc;
  rows->seq_slots = seq_slots;
  rows->tables = tables;
  rows->nblk = nblk;
  rows->max_seqs = static_cast<int32_t>(pool->max_seqs);
  rows->width = static_cast<int32_t>(pool->max_blocks_per_seq);
  return NKV_OK;
}

}  // namespace

extern "C" int nkv_pack_decode_pool(const nkv_pool_desc* pool, const int32_t* num_tokens,
                                    const int32_t* seq_slots, int64_t num_seqs,
                                    int64_t padded_seqs, int64_t block_size,
                                    int64_t table_width, int64_t table_stride,
                                    int32_t* slot_mapping, int32_t* context_lens,
                                    int32_t* block_tables, int32_t* cu_seqlens_k,
                                    void* stream) {
  using namespace nkv;
  PoolRows rows{};
  if (int rc = pool_rows(pool, seq_slots, "nkv_pack_decode_pool", &rows)) return rc;
  if (int rc = check_pack_args("nkv_pack_decode_pool", 0, num_seqs, block_size, table_width)) {
    return rc;
  }
  if (padded_seqs < num_seqs || padded_seqs > NKV_MAX_PACK_SEQS || table_stride < table_width) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_pack_decode_pool: padded_seqs must be in [num_seqs, %d] and "
                    "table_stride >= table_width",
                    NKV_MAX_PACK_SEQS);
  }
  if (padded_seqs == 0 && cu_seqlens_k == nullptr) return NKV_OK;
  if ((padded_seqs > 0 && !slot_mapping) || (num_seqs > 0 && (!num_tokens || !seq_slots))) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_decode_pool: null pointer");
  }
  const size_t lds = cu_seqlens_k != nullptr
                         ? (static_cast<size_t>(num_seqs) + 1 + kPackWaves + 1) * sizeof(int32_t)
                         : 0;
  pack_decode_kernel<<<dim3(pack_grid(padded_seqs, 0)), dim3(kPackThreads), lds,
                       static_cast<hipStream_t>(stream)>>>(
      num_tokens, rows, static_cast<int32_t>(num_seqs), static_cast<int32_t>(padded_seqs),
      static_cast<int32_t>(block_size), static_cast<int32_t>(table_width), table_stride,
      slot_mapping, context_lens, block_tables, cu_seqlens_k);
  return nkv_check_launch("nkv_pack_decode_pool");
}

extern "C" int nkv_pack_prefill_pool(const nkv_pool_desc* pool, const int32_t* num_cached,
                                     const int32_t* num_scheduled, const int32_t* num_prompt,
                                     const int32_t* seq_slots, int64_t num_seqs,
                                     int64_t block_size, int64_t table_width, int64_t num_slots,
                                     int32_t* cu_seqlens_q, int32_t* cu_seqlens_k,
                                     int32_t* slot_mapping, int32_t* block_tables,
                                     int32_t* full_context_lens, int32_t* query_start_lens,
                                     int32_t* max_seqlens, void* stream) {
  using namespace nkv;
  PoolRows rows{};
  if (int rc = pool_rows(pool, seq_slots, "nkv_pack_prefill_pool", &rows)) return rc;
  if (int rc = check_pack_args("nkv_pack_prefill_pool", 0, num_seqs, block_size, table_width)) {
    return rc;
  }
  if (num_slots < 0 || num_slots > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_prefill_pool: num_slots out of range");
  }
  if ((num_seqs > 0 && (!num_cached || !num_scheduled || !seq_slots)) ||
      (num_slots > 0 && !slot_mapping) || (full_context_lens && !num_prompt)) {
    return nkv_fail(NKV_E_INVALID, "nkv_pack_prefill_pool: null pointer");
  }
  const size_t lds =
      (2 * (static_cast<size_t>(num_seqs) + 1) + 3 * kPackWaves + 1) * sizeof(int32_t);
  pack_prefill_kernel<<<dim3(pack_grid(num_seqs, num_slots)), dim3(kPackThreads), lds,
                        static_cast<hipStream_t>(stream)>>>(
      num_cached, num_scheduled, num_prompt, rows, static_cast<int32_t>(num_seqs),
      static_cast<int32_t>(block_size), static_cast<int32_t>(table_width),
      static_cast<int32_t>(num_slots), cu_seqlens_q, cu_seqlens_k, slot_mapping, block_tables,
      full_context_lens, query_start_lens, max_seqlens);
  return nkv_check_launch("nkv_pack_prefill_pool");
}
