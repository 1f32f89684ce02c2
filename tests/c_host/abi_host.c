/*
 * A C host program that drives libnanokv through its C ABI alone: its own
 * hipMalloc'd buffers and its own stream, no Python and no torch, the way a
 * non-Python caller of the reference's store/gather ops (an FFI binding)
 * would.  Every output is compared byte for byte with the oracle's C
 * restatement (oracle/nkv_oracle.c, test infrastructure linked as the
 * checker).
 *
 * Cases: a bf16 store of 300 tokens into 96 blocks of 16 rows (two -1
 * slots), then the varlen K/V gather of six contexts (0, 1, 15, 16, 17 and
 * 700 rows) through nkv_gather_varlen with a caller workspace and through
 * nkv_gather_varlen_noalloc, the single-sequence nkv_gather of the longest
 * context, and one contract violation (a NULL key) that must return
 * NKV_E_INVALID with a message.  Prints "abi_host ok" and exits 0 when all
 * match; exits 1 on a mismatch, 2 when no GPU is visible.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <hip/hip_runtime_api.h>

#include "nanokv.h"

/* oracle/nkv_oracle.c */
void nkvo_store(const uint8_t* key, const uint8_t* value, uint8_t* key_cache,
                uint8_t* value_cache, const int32_t* slots, int64_t num_tokens,
                int64_t key_stride_bytes, int64_t value_stride_bytes, int64_t row_bytes,
                int threads);
void nkvo_gather(const uint8_t* cache, const int32_t* table, int64_t len, int64_t block_size,
                 int64_t row_bytes, uint8_t* out, int threads);
void nkvo_gather_varlen(const uint8_t* cache, const int32_t* tables, int64_t table_stride,
                        const int32_t* cu, int64_t num_seqs, int64_t block_size,
                        int64_t row_bytes, uint8_t* out, int threads);

#define NUM_BLOCKS 96
#define BLOCK_SIZE 16
#define ROW_ELEMS (8 * 128) /* 8 kv heads x head_dim 128 */
#define ROW_BYTES (ROW_ELEMS * 2)
#define NUM_TOKENS 300
#define NUM_SEQS 6

#define HIP_OK(call)                                                              \
  do {                                                                            \
    hipError_t err_ = (call);                                                     \
    if (err_ != hipSuccess) {                                                     \
      fprintf(stderr, "abi_host: %s failed: %s\n", #call, hipGetErrorString(err_)); \
      exit(1);                                                                    \
    }                                                                             \
  } while (0)

#define NKV_OK_CALL(call)                                                         \
  do {                                                                            \
    int rc_ = (call);                                                             \
    if (rc_ != NKV_OK) {                                                          \
      fprintf(stderr, "abi_host: %s returned %d: %s\n", #call, rc_, nkv_last_error()); \
      exit(1);                                                                    \
    }                                                                             \
  } while (0)

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;

static uint32_t next_u32(void) { /* xorshift64* */
  rng_state ^= rng_state >> 12;
  rng_state ^= rng_state << 25;
  rng_state ^= rng_state >> 27;
  return (uint32_t)((rng_state * 0x2545F4914F6CDD1Dull) >> 32);
}

static void fill_words(uint8_t* p, size_t bytes) {
  for (size_t i = 0; i + 4 <= bytes; i += 4) {
    const uint32_t w = next_u32();
    memcpy(p + i, &w, 4);
  }
}

/* The first n entries of a random permutation of [0, range). */
static void permutation(int32_t* out, int32_t n, int32_t range) {
  int32_t* all = malloc(sizeof(int32_t) * (size_t)range);
  for (int32_t i = 0; i < range; ++i) all[i] = i;
  for (int32_t i = range - 1; i > 0; --i) {
    const int32_t j = (int32_t)(next_u32() % (uint32_t)(i + 1));
    const int32_t t = all[i];
    all[i] = all[j];
    all[j] = t;
  }
  memcpy(out, all, sizeof(int32_t) * (size_t)n);
  free(all);
}

static void* device_copy(const void* host, size_t bytes) {
  void* d = NULL;
  HIP_OK(hipMalloc(&d, bytes > 0 ? bytes : 16));
  if (bytes > 0) HIP_OK(hipMemcpy(d, host, bytes, hipMemcpyHostToDevice));
  return d;
}

static int same(const char* what, const void* got, const void* want, size_t bytes) {
  if (memcmp(got, want, bytes) == 0) return 1;
  const uint8_t* g = got;
  const uint8_t* w = want;
  size_t i = 0;
  while (i < bytes && g[i] == w[i]) ++i;
  fprintf(stderr, "abi_host: %s differs from the oracle at byte %zu of %zu\n", what, i, bytes);
  return 0;
}

int main(void) {
  int devices = 0;
  if (hipGetDeviceCount(&devices) != hipSuccess || devices < 1) {
    fprintf(stderr, "abi_host: no GPU visible\n");
    return 2;
  }
  HIP_OK(hipSetDevice(0));
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));

  const size_t cache_bytes = (size_t)NUM_BLOCKS * BLOCK_SIZE * ROW_BYTES;
  const size_t token_bytes = (size_t)NUM_TOKENS * ROW_BYTES;
  uint8_t* key = malloc(token_bytes);
  uint8_t* value = malloc(token_bytes);
  uint8_t* key_cache = malloc(cache_bytes);
  uint8_t* value_cache = malloc(cache_bytes);
  fill_words(key, token_bytes);
  fill_words(value, token_bytes);
  fill_words(key_cache, cache_bytes);
  fill_words(value_cache, cache_bytes);
  int32_t slots[NUM_TOKENS];
  permutation(slots, NUM_TOKENS, NUM_BLOCKS * BLOCK_SIZE);
  slots[7] = -1;
  slots[150] = -1;

  /* six contexts over distinct blocks, tables padded with -1 */
  const int32_t lens[NUM_SEQS] = {0, 1, 15, 16, 17, 700};
  const int32_t width = (700 + BLOCK_SIZE - 1) / BLOCK_SIZE;
  int32_t tables[NUM_SEQS * ((700 + BLOCK_SIZE - 1) / BLOCK_SIZE)];
  int32_t order[NUM_BLOCKS];
  permutation(order, NUM_BLOCKS, NUM_BLOCKS);
  int32_t cu[NUM_SEQS + 1];
  cu[0] = 0;
  int32_t next_block = 0;
  for (int i = 0; i < NUM_SEQS; ++i) {
    const int32_t need = (lens[i] + BLOCK_SIZE - 1) / BLOCK_SIZE;
    for (int32_t b = 0; b < width; ++b) tables[i * width + b] = b < need ? order[next_block + b] : -1;
    next_block += need;
    cu[i + 1] = cu[i] + lens[i];
  }
  const int64_t total = cu[NUM_SEQS];

  uint8_t* d_key = device_copy(key, token_bytes);
  uint8_t* d_value = device_copy(value, token_bytes);
  uint8_t* d_kc = device_copy(key_cache, cache_bytes);
  uint8_t* d_vc = device_copy(value_cache, cache_bytes);
  int32_t* d_slots = device_copy(slots, sizeof(slots));
  int32_t* d_tables = device_copy(tables, sizeof(tables));
  int32_t* d_cu = device_copy(cu, sizeof(cu));
  const size_t out_bytes = (size_t)total * ROW_BYTES;
  uint8_t *d_kout = NULL, *d_vout = NULL, *d_kout2 = NULL, *d_vout2 = NULL, *d_one = NULL;
  HIP_OK(hipMalloc((void**)&d_kout, out_bytes));
  HIP_OK(hipMalloc((void**)&d_vout, out_bytes));
  HIP_OK(hipMalloc((void**)&d_kout2, out_bytes));
  HIP_OK(hipMalloc((void**)&d_vout2, out_bytes));
  HIP_OK(hipMalloc((void**)&d_one, (size_t)lens[5] * ROW_BYTES));

  NKV_OK_CALL(nkv_store(d_key, d_value, d_kc, d_vc, d_slots, NUM_TOKENS, ROW_ELEMS, ROW_ELEMS,
                        ROW_ELEMS, NUM_BLOCKS * BLOCK_SIZE, NKV_DTYPE_BFLOAT16, stream));
  const int64_t capacity =
      nkv_gather_plan_capacity(total, NUM_SEQS, BLOCK_SIZE, ROW_ELEMS, NKV_DTYPE_BFLOAT16);
  if (capacity <= 0) {
    fprintf(stderr, "abi_host: nkv_gather_plan_capacity returned %lld\n", (long long)capacity);
    return 1;
  }
  void* d_workspace = NULL;
  HIP_OK(hipMalloc(&d_workspace, (size_t)capacity * 16));
  NKV_OK_CALL(nkv_gather_varlen(d_kc, d_vc, d_tables, width, d_cu, NUM_SEQS, total, BLOCK_SIZE,
                                ROW_ELEMS, NUM_BLOCKS, NKV_DTYPE_BFLOAT16, d_kout, d_vout,
                                d_workspace, capacity * 16, stream));
  NKV_OK_CALL(nkv_gather_varlen_noalloc(d_kc, d_vc, d_tables, width, d_cu, NUM_SEQS, total,
                                        BLOCK_SIZE, ROW_ELEMS, NUM_BLOCKS, NKV_DTYPE_BFLOAT16,
                                        d_kout2, d_vout2, stream));
  NKV_OK_CALL(nkv_gather(d_kc, d_tables + 5 * width, width, lens[5], BLOCK_SIZE, ROW_ELEMS,
                         NUM_BLOCKS, NKV_DTYPE_BFLOAT16, d_one, stream));
  HIP_OK(hipStreamSynchronize(stream));

  /* a contract violation is rejected on the host with a message */
  const int bad = nkv_store(NULL, d_value, d_kc, d_vc, d_slots, 5, ROW_ELEMS, ROW_ELEMS,
                            ROW_ELEMS, NUM_BLOCKS * BLOCK_SIZE, NKV_DTYPE_BFLOAT16, stream);
  const char* message = nkv_last_error();
  if (bad != NKV_E_INVALID || message == NULL || message[0] == '\0') {
    fprintf(stderr, "abi_host: a NULL key returned %d (message '%s'), expected NKV_E_INVALID\n",
            bad, message ? message : "(null)");
    return 1;
  }

  uint8_t* got_kc = malloc(cache_bytes);
  uint8_t* got_vc = malloc(cache_bytes);
  uint8_t* got_k = malloc(out_bytes);
  uint8_t* got_v = malloc(out_bytes);
  uint8_t* got_k2 = malloc(out_bytes);
  uint8_t* got_v2 = malloc(out_bytes);
  uint8_t* got_one = malloc((size_t)lens[5] * ROW_BYTES);
  HIP_OK(hipMemcpy(got_kc, d_kc, cache_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(got_vc, d_vc, cache_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(got_k, d_kout, out_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(got_v, d_vout, out_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(got_k2, d_kout2, out_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(got_v2, d_vout2, out_bytes, hipMemcpyDeviceToHost));
  HIP_OK(hipMemcpy(got_one, d_one, (size_t)lens[5] * ROW_BYTES, hipMemcpyDeviceToHost));

  /* the oracle: the same store on the host caches, then the gathers */
  nkvo_store(key, value, key_cache, value_cache, slots, NUM_TOKENS, ROW_BYTES, ROW_BYTES,
             ROW_BYTES, 1);
  uint8_t* want_k = malloc(out_bytes);
  uint8_t* want_v = malloc(out_bytes);
  uint8_t* want_one = malloc((size_t)lens[5] * ROW_BYTES);
  nkvo_gather_varlen(key_cache, tables, width, cu, NUM_SEQS, BLOCK_SIZE, ROW_BYTES, want_k, 1);
  nkvo_gather_varlen(value_cache, tables, width, cu, NUM_SEQS, BLOCK_SIZE, ROW_BYTES, want_v, 1);
  nkvo_gather(key_cache, tables + 5 * width, lens[5], BLOCK_SIZE, ROW_BYTES, want_one, 1);

  int ok = 1;
  ok &= same("key cache after nkv_store", got_kc, key_cache, cache_bytes);
  ok &= same("value cache after nkv_store", got_vc, value_cache, cache_bytes);
  ok &= same("K of nkv_gather_varlen", got_k, want_k, out_bytes);
  ok &= same("V of nkv_gather_varlen", got_v, want_v, out_bytes);
  ok &= same("K of nkv_gather_varlen_noalloc", got_k2, want_k, out_bytes);
  ok &= same("V of nkv_gather_varlen_noalloc", got_v2, want_v, out_bytes);
  ok &= same("nkv_gather of the 700-row context", got_one, want_one, (size_t)lens[5] * ROW_BYTES);

  HIP_OK(hipFree(d_key));
  HIP_OK(hipFree(d_value));
  HIP_OK(hipFree(d_kc));
  HIP_OK(hipFree(d_vc));
  HIP_OK(hipFree(d_slots));
  HIP_OK(hipFree(d_tables));
  HIP_OK(hipFree(d_cu));
  HIP_OK(hipFree(d_kout));
  HIP_OK(hipFree(d_vout));
  HIP_OK(hipFree(d_kout2));
  HIP_OK(hipFree(d_vout2));
  HIP_OK(hipFree(d_one));
  HIP_OK(hipFree(d_workspace));
  HIP_OK(hipStreamDestroy(stream));
  free(key);
  free(value);
  free(key_cache);
  free(value_cache);
  free(got_kc);
  free(got_vc);
  free(got_k);
  free(got_v);
  free(got_k2);
  free(got_v2);
  free(got_one);
  free(want_k);
  free(want_v);
  free(want_one);
  if (!ok) return 1;
  printf("abi_host ok: store, gather_varlen (workspace and no-alloc), gather and a rejected "
         "NULL key match the oracle (%lld context rows)\n", (long long)total);
  return 0;
}
