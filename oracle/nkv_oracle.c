/*
 * CPU restatement of the reference's paged-KV hot path in plain C.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg (to check results, and as the timed CPU baseline),
 * never by the product.  Rows are opaque byte strings (row_bytes =
 * kv_heads*head_dim*element size), so results are bit-exact by construction.
 * Loops over tokens / blocks / sequences run under OpenMP with `threads`
 * threads; outputs are disjoint per iteration when slots are unique, the
 * contract of the reference (nanovllm/layers/attention.py:24-25).
 */
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* nanovllm/layers/paged_kv/pytorch_backend.py:26-38: skip slot < 0, else
 * copy key row t and value row t to cache row slot. */
void nkvo_store(const uint8_t* key, const uint8_t* value, uint8_t* key_cache,
                uint8_t* value_cache, const int32_t* slots, int64_t num_tokens,
                int64_t key_stride_bytes, int64_t value_stride_bytes,
                int64_t row_bytes, int threads) {
  int64_t t;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (t = 0; t < num_tokens; ++t) {
    const int64_t slot = slots[t];
    if (slot < 0) continue;
    memcpy(key_cache + slot * row_bytes, key + t * key_stride_bytes, (size_t)row_bytes);
    memcpy(value_cache + slot * row_bytes, value + t * value_stride_bytes, (size_t)row_bytes);
  }
}

/* pytorch_backend.py:40-50: out[t] = cache row (table[t/BS], t%BS) for
 * t < L, one memcpy per logical block (the rows of a block are
 * contiguous). */
static void gather_one(const uint8_t* cache, const int32_t* table, int64_t len,
                       int64_t block_size, int64_t row_bytes, uint8_t* out) {
  const int64_t blocks = (len + block_size - 1) / block_size;
  for (int64_t b = 0; b < blocks; ++b) {
    const int64_t rows = (len - b * block_size) < block_size ? (len - b * block_size) : block_size;
    memcpy(out + b * block_size * row_bytes,
           cache + (int64_t)table[b] * block_size * row_bytes,
           (size_t)(rows * row_bytes));
  }
}

void nkvo_gather(const uint8_t* cache, const int32_t* table, int64_t len,
                 int64_t block_size, int64_t row_bytes, uint8_t* out, int threads) {
  const int64_t blocks = (len + block_size - 1) / block_size;
  int64_t b;
#pragma omp parallel for num_threads(threads) schedule(static)
  for (b = 0; b < blocks; ++b) {
    const int64_t rows = (len - b * block_size) < block_size ? (len - b * block_size) : block_size;
    memcpy(out + b * block_size * row_bytes,
           cache + (int64_t)table[b] * block_size * row_bytes,
           (size_t)(rows * row_bytes));
  }
}

/* Concatenation of per-request gathers (nanovllm/layers/attention.py:
 * 250-259, 284-292): request i lands at row cu[i] and has cu[i+1]-cu[i]
 * rows. */
void nkvo_gather_varlen(const uint8_t* cache, const int32_t* tables,
                        int64_t table_stride, const int32_t* cu,
                        int64_t num_seqs, int64_t block_size, int64_t row_bytes,
                        uint8_t* out, int threads) {
  int64_t i;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (i = 0; i < num_seqs; ++i) {
    gather_one(cache, tables + i * table_stride, (int64_t)cu[i + 1] - cu[i],
               block_size, row_bytes, out + (int64_t)cu[i] * row_bytes);
  }
}

/* model_runner.py:892-938 + :696-707 + sequence.py:176-183. */
void nkvo_pack_decode(const int32_t* num_tokens, const int32_t* offsets,
                      const int32_t* ids, int64_t num_seqs, int64_t block_size,
                      int64_t width, int32_t* slots, int32_t* context_lens,
                      int32_t* tables, int32_t* cu_seqlens_k) {
  int64_t running = 0;
  for (int64_t i = 0; i < num_seqs; ++i) {
    const int64_t n = num_tokens[i];
    const int64_t count = offsets[i + 1] - offsets[i];
    const int64_t blocks = (n + block_size - 1) / block_size;
    const int64_t last_tokens = n - (blocks - 1) * block_size;
    slots[i] = (int32_t)(ids[offsets[i + 1] - 1] * block_size + last_tokens - 1);
    context_lens[i] = (int32_t)n;
    for (int64_t j = 0; j < width; ++j) {
      tables[i * width + j] = j < count ? ids[offsets[i] + j] : -1;
    }
    if (cu_seqlens_k) cu_seqlens_k[i] = (int32_t)running;
    running += n;
  }
  if (cu_seqlens_k) cu_seqlens_k[num_seqs] = (int32_t)running;
}

/* model_runner.py:757-820 (slots, cu_seqlens, starts), closed form
 * slot(p) = bt[p/BS]*BS + p%BS over p in [start, end). */
void nkvo_pack_prefill(const int32_t* num_cached, const int32_t* num_scheduled,
                       const int32_t* offsets, const int32_t* ids,
                       int64_t num_seqs, int64_t block_size, int64_t width,
                       int32_t* cu_q, int32_t* cu_k, int32_t* slots,
                       int32_t* tables) {
  int64_t q_run = 0, k_run = 0, s_run = 0;
  for (int64_t i = 0; i < num_seqs; ++i) {
    const int64_t start = num_cached[i];
    const int64_t end = start + num_scheduled[i];
    const int64_t count = offsets[i + 1] - offsets[i];
    cu_q[i] = (int32_t)q_run;
    cu_k[i] = (int32_t)k_run;
    q_run += num_scheduled[i];
    k_run += end;
    if (count > 0) {
      for (int64_t p = start; p < end; ++p) {
        slots[s_run++] = (int32_t)(ids[offsets[i] + p / block_size] * block_size + p % block_size);
      }
    }
    if (tables) {
      for (int64_t j = 0; j < width; ++j) {
        tables[i * width + j] = j < count ? ids[offsets[i] + j] : -1;
      }
    }
  }
  cu_q[num_seqs] = (int32_t)q_run;
  cu_k[num_seqs] = (int32_t)k_run;
}

int nkvo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
