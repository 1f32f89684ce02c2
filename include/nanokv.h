/*
 * nanokv — paged KV-cache store / gather / ragged-batch metadata packing for
 * AMD Instinct MI355X (gfx950).  Plain C ABI: device pointers, int64 sizes,
 * an opaque stream handle (a hipStream_t; NULL = the legacy default stream).
 *
 * Every entry point is asynchronous on `stream`, returns 0 on success and a
 * non-zero NKV_E* code on failure; nkv_last_error() then returns a message
 * (thread-local, valid until the next call on the same thread).  Contract
 * violations that the host can see without reading device memory (negative
 * sizes, misaligned pointers for the dtype, capacity too small) are rejected
 * before any launch.  Index VALUES living in device memory (slots, physical
 * block ids) are never trusted by the kernels: a slot outside [0, num_slots)
 * is skipped like the -1 padding slot, and a physical block outside
 * [0, num_blocks) yields zero-filled output rows, so a bad index can never
 * fault the GPU.  Range validation that raises is the host's job (the Python
 * validators, behind NANOVLLM_PAGED_KV_VALIDATE_INDICES as in the reference).
 *
 * Layouts (all row-major / contiguous unless a stride says otherwise):
 *   cache         [num_blocks, block_size, kv_heads, head_dim]; one "row" is
 *                 one (block, slot) = row_elems = kv_heads*head_dim elements.
 *   key / value   [num_tokens, kv_heads, head_dim] with an arbitrary token
 *                 stride (fused-QKV views) and contiguous inner dims.
 *   block_tables  [num_seqs, table_stride] int32, -1 padded, contiguous
 *                 (table_stride is both the row stride and the width).
 *   cu_seqlens    [num_seqs + 1] int32 exclusive prefix sums.
 *
 * dtype selects only the element size (the kernels move bits, never convert).
 */
#ifndef NANOKV_H
#define NANOKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes: the three dtypes the reference dispatches on
 * (AT_DISPATCH_FLOATING_TYPES_AND2(Half, BFloat16) in
 * csrc/paged_kv/paged_kv_cuda.cu:115-117 and :149-151). */
#define NKV_DTYPE_FLOAT16 0
#define NKV_DTYPE_BFLOAT16 1
#define NKV_DTYPE_FLOAT32 2

/* error codes */
#define NKV_OK 0
#define NKV_E_INVALID 1   /* bad argument (host-visible contract violation) */
#define NKV_E_HIP 2       /* a HIP runtime call failed                      */
#define NKV_E_CAPACITY 3  /* caller buffer / limit too small                */

/* Library version (major*10000 + minor*100 + patch). */
int nkv_version(void);

/*
 * Build id: "<sources>-<config>", where <sources> is 16 hex digits of a
 * SHA-256 over every source and header file, the compiler flags and the
 * offload architecture, and <config> is "default" or 8 hex digits of the
 * launch-shape defines the library was compiled with.  A loader recomputes
 * <sources> from the files on disk and refuses a library that differs.
 *
 * Replaces: the reference's build fingerprint, which names the extension
 *   build after a SHA-256 of its sources, flags, toolchain and arch list so
 *   that a changed source rebuilds it (nanovllm/layers/paged_kv/
 *   loader.py:47-85, tested in tests/test_paged_kv_extension_loader.py:12-32).
 */
const char* nkv_build_id(void);

/* Message for the last failing call on this thread ("" if none). */
const char* nkv_last_error(void);

/*
 * Store: for every token t with 0 <= slot_mapping[t] < num_slots, copy the
 * key row t into key_cache row slot_mapping[t] and the value row t into
 * value_cache row slot_mapping[t]; slot -1 (and any other out-of-range slot)
 * is skipped.  num_tokens == 0 is a no-op.
 *
 * Replaces: the op `nanovllm_paged_kv::store(Tensor key, Tensor value,
 *   Tensor(a!) key_cache, Tensor(b!) value_cache, Tensor slot_mapping) -> ()`
 *   (csrc/paged_kv/paged_kv.cpp:200-201), whose CUDA implementation is
 *   store_cuda (csrc/paged_kv/paged_kv_cuda.cu:96-132); semantics of the
 *   pytorch oracle nanovllm/layers/paged_kv/pytorch_backend.py:26-38.
 * Strides are in elements (key.stride(0), value.stride(0)); row_elems is
 * kv_heads*head_dim (key.size(1)*key.size(2)), and a token's row_elems
 * elements must be contiguous (a view strided between heads is compacted by
 * the caller first); num_slots is num_blocks*block_size of the cache.
 */
int nkv_store(const void* key, const void* value, void* key_cache,
              void* value_cache, const int32_t* slot_mapping,
              int64_t num_tokens, int64_t key_token_stride,
              int64_t value_token_stride, int64_t row_elems,
              int64_t num_slots, int32_t dtype, void* stream);

/*
 * Gather one sequence: out[t] = cache row (block_table[t / block_size],
 * t % block_size) for t in [0, sequence_length).  out is a contiguous
 * [sequence_length, row_elems] buffer owned by the caller.
 *
 * Replaces: the op `nanovllm_paged_kv::gather(Tensor cache,
 *   Tensor block_table, int sequence_length) -> Tensor`
 *   (csrc/paged_kv/paged_kv.cpp:202), CUDA implementation gather_cuda
 *   (csrc/paged_kv/paged_kv_cuda.cu:134-164); pytorch oracle
 *   nanovllm/layers/paged_kv/pytorch_backend.py:40-50.  The output
 *   allocation the reference op performs (at::empty, :142-143) is done by
 *   the caller here, so the ABI never allocates.  table_len (entries of
 *   block_table) must cover ceil(sequence_length / block_size) blocks, the
 *   check of nanovllm/layers/paged_kv/base.py:138-139.
 */
int nkv_gather(const void* cache, const int32_t* block_table,
               int64_t table_len, int64_t sequence_length, int64_t block_size,
               int64_t row_elems, int64_t num_blocks, int32_t dtype,
               void* out, void* stream);

/*
 * Gather plans.  A plan splits every sequence's context into chunks of
 * `chunk_rows` consecutive rows that never cross a cache block, one int4
 * entry {src_row, dst_row, num_rows, seq} per chunk; it depends only on the
 * block tables and cu_seqlens_k, so one plan serves both caches of every
 * layer in a decode step.  Entries past the real chunk count have
 * num_rows = 0.  src_row = -1 marks a chunk whose physical block is outside
 * [0, num_blocks) (rows come out zero-filled).
 *
 * nkv_gather_plan_rows: the chunk length (rows) the library uses for a row
 *   size and block size (a divisor of block_size).
 * nkv_gather_plan_capacity: entries needed for total_rows rows spread over
 *   num_seqs sequences (an upper bound, ceil(total_rows/chunk)+num_seqs).
 */
int64_t nkv_gather_plan_rows(int64_t block_size, int64_t row_elems,
                             int32_t dtype);
int64_t nkv_gather_plan_capacity(int64_t total_rows, int64_t num_seqs,
                                 int64_t block_size, int64_t row_elems,
                                 int32_t dtype);

/*
 * Build a gather plan on the device from block_tables [num_seqs,
 * table_stride] and cu_seqlens_k [num_seqs+1] (context lengths are
 * cu_seqlens_k[i+1]-cu_seqlens_k[i]).  plan must hold `capacity` int4
 * entries (16 B each, 16-B aligned); capacity must be at least
 * nkv_gather_plan_capacity(cu_seqlens_k[num_seqs], ...).  num_seqs is
 * limited to NKV_MAX_PLAN_SEQS.  out_rows is the row count of the outputs
 * the plan will be used with: chunks outside [0, out_rows) are clipped, and
 * a logical block at or past table_stride reads as invalid, so wrong
 * device-side lengths cannot make the gather write or read out of bounds.
 *
 * No reference counterpart as a single call: it replaces the per-request
 * host loop of SDPAAttention (nanovllm/layers/attention.py:250-259 prefill,
 * :284-292 decode) that issues one gather launch per (request, K or V).
 */
#define NKV_MAX_PLAN_SEQS 8192
int nkv_build_gather_plan(const int32_t* block_tables, int64_t table_stride,
                          const int32_t* cu_seqlens_k, int64_t num_seqs,
                          int64_t out_rows, int64_t block_size, int64_t row_elems,
                          int64_t num_blocks, int32_t dtype, void* plan,
                          int64_t capacity, void* stream);

/*
 * Varlen gather of K and V for every sequence with one launch, driven by a
 * plan from nkv_build_gather_plan (same block_size/row_elems/dtype):
 * key_out[cu_seqlens_k[i] + t] = key_cache row of token t of sequence i,
 * likewise for V.  Equals, byte for byte, the concatenation over i of the
 * reference's gather(cache, block_tables[i], context_len[i])
 * (nanovllm/layers/attention.py:254-259, :287-292).
 * value_cache / value_out may be NULL together to gather one cache only.
 * cache_rows (num_blocks*block_size of each cache) and out_rows (rows of
 * each output) bound every entry: an entry reaching past the cache is
 * zero-filled, one reaching past the output is skipped, so the launch stays
 * in bounds whatever plan it is given.
 */
int nkv_gather_varlen_planned(const void* key_cache, const void* value_cache,
                              const void* plan, int64_t capacity,
                              int64_t cache_rows, int64_t out_rows,
                              int64_t block_size, int64_t row_elems,
                              int32_t dtype,
                              void* key_out, void* value_out, void* stream);

/*
 * Convenience: build the plan into `workspace` (workspace_bytes >=
 * 16*capacity) and run the planned gather, two launches.
 */
int nkv_gather_varlen(const void* key_cache, const void* value_cache,
                      const int32_t* block_tables, int64_t table_stride,
                      const int32_t* cu_seqlens_k, int64_t num_seqs,
                      int64_t total_rows, int64_t block_size,
                      int64_t row_elems, int64_t num_blocks, int32_t dtype,
                      void* key_out, void* value_out, void* workspace,
                      int64_t workspace_bytes, void* stream);

/*
 * Prefill store + context gather in one launch: the result of nkv_store
 * followed by the varlen gather of every request's whole context, with each
 * new row read once.  Request i has Lq = cu_seqlens_q[i+1] - cu_seqlens_q[i]
 * new tokens (rows cu_seqlens_q[i].. of key / value and slot_mapping), which
 * are the last Lq of its Lk = cu_seqlens_k[i+1] - cu_seqlens_k[i] context
 * positions; key_out / value_out [out_rows, row_elems] receive context row p
 * of request i at cu_seqlens_k[i] + p, as nkv_gather_varlen does.  The
 * caches are updated exactly as nkv_store updates them.
 *
 * Exactness condition (what the reference's packing and scheduling
 * produce): no two tokens share a slot, a token's slot is -1 or the
 * table-derived slot of its own position (model_runner.py:757-820), and no
 * request's cached prefix, positions [0, Lk - Lq), holds a row that a token
 * of this call stores.  The reference guarantees the last: a block enters
 * the prefix cache only after the step that filled it (Scheduler.postprocess
 * -> BlockManager.hash_blocks, nanovllm/engine/scheduler.py:196-200,
 * block_manager.py:229-258), so a request of a step never finds its prefix
 * in rows that step writes.  A token whose slot is -1 or differs is stored
 * as given, and its output row is read from the cache row of its position,
 * as the gather finds it (the reference's store already forbids duplicate
 * slots, attention.py:24-25).  A batch that breaks the last condition gets
 * unspecified values in the output rows concerned (never an access outside
 * the buffers); nkv_store followed by nkv_gather_varlen handles it.
 *
 * Replaces: the store call of Attention.forward (nanovllm/layers/
 *   attention.py:87-93) together with the per-request gathers of
 *   SDPAAttention's prefill (attention.py:250-259), as one launch.
 *
 * nkv_store_gather_plan_bytes: bytes of the per-step plan (16 per chunk of
 *   cached rows, 8 per token).
 * nkv_build_store_gather_plan: builds it on the device (one launch) from
 *   block_tables [num_seqs, table_stride], cu_seqlens_q and cu_seqlens_k
 *   (num_seqs at most NKV_MAX_PACK_SEQS); num_tokens is the step's rows of
 *   key / value / slot_mapping (cu_seqlens_q[num_seqs]) and out_rows its
 *   context rows (cu_seqlens_k[num_seqs]).  One plan serves every layer.
 * nkv_store_gather: the launch.  plan_bytes must be exactly what
 *   nkv_store_gather_plan_bytes returns for this call's num_tokens,
 *   out_rows, num_seqs and geometry (a plan built for other counts is
 *   rejected with NKV_E_CAPACITY).  Every index the kernel reads from device
 *   memory is bounded by the buffers, whatever the plan holds.
 */
int64_t nkv_store_gather_plan_bytes(int64_t num_tokens, int64_t total_rows,
                                    int64_t num_seqs, int64_t block_size,
                                    int64_t row_elems, int32_t dtype);
int nkv_build_store_gather_plan(const int32_t* block_tables, int64_t table_stride,
                                const int32_t* cu_seqlens_q,
                                const int32_t* cu_seqlens_k, int64_t num_seqs,
                                int64_t num_tokens, int64_t out_rows,
                                int64_t block_size, int64_t row_elems,
                                int64_t num_blocks, int32_t dtype, void* plan,
                                int64_t plan_bytes, void* stream);
int nkv_store_gather(const void* key, const void* value, void* key_cache,
                     void* value_cache, const int32_t* slot_mapping,
                     int64_t num_tokens, int64_t key_token_stride,
                     int64_t value_token_stride, const void* plan,
                     int64_t plan_bytes, int64_t num_seqs, int64_t out_rows,
                     int64_t block_size, int64_t row_elems, int64_t num_blocks,
                     int32_t dtype, void* key_out, void* value_out, void* stream);

/*
 * nkv_gather_varlen without a workspace, for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops and harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Same arguments
 * and result as nkv_gather_varlen minus the workspace: the plan lives in a
 * device array inside the library (NKV_SCRATCH_BYTES per GPU, held until
 * the process ends), so the call allocates nothing.  A plan larger than the
 * array (nkv_gather_plan_capacity(...) * 16 > NKV_SCRATCH_BYTES, i.e. about
 * 4.2 million rows of 2 KiB) is rejected with NKV_E_CAPACITY before any
 * device work.  The device is the calling thread's current device, which
 * must own `stream`.  Every call on one GPU uses that GPU's one array:
 * calls that overlap on the same GPU (different streams without ordering,
 * or concurrent threads) race and must not be issued; calls on one stream
 * are ordered and safe.
 */
#define NKV_SCRATCH_BYTES (4 << 20)
int nkv_gather_varlen_noalloc(const void* key_cache, const void* value_cache,
                              const int32_t* block_tables, int64_t table_stride,
                              const int32_t* cu_seqlens_k, int64_t num_seqs,
                              int64_t total_rows, int64_t block_size,
                              int64_t row_elems, int64_t num_blocks,
                              int32_t dtype, void* key_out, void* value_out,
                              void* stream);

/*
 * Decode-step metadata packing on the device.  Input is the scheduler's
 * per-sequence state in CSR form: num_tokens[i] (len(seq)), and the block
 * list of sequence i = block_ids[block_offsets[i] .. block_offsets[i+1]);
 * num_block_ids is the length of block_ids (reads past it yield -1).
 * Outputs (all int32, device):
 *   slot_mapping[i]  = last_block*block_size + last_block_num_tokens - 1
 *                      (-1 when the block list is empty)
 *   context_lens[i]  = num_tokens[i]                          (may be NULL)
 *   block_tables     rows of table_stride entries: columns [0, table_width)
 *                    of rows [0, num_seqs) get the block list, -1 padded;
 *                    table_width must be >= the longest block list, and
 *                    columns >= table_width keep their contents (may be NULL)
 *   cu_seqlens_k     [padded_seqs+1], exclusive prefix sum of num_tokens
 *                    (may be NULL)
 * Rows [num_seqs, padded_seqs) are graph-bucket padding: slot -1, context
 * length 0, cu_seqlens_k flat, block-table rows untouched.  Writing into
 * fixed buffers this way reproduces the decode graph's replay fill
 * (model_runner.py:993-1011) without the -1/0 fills and D2D copies.
 *
 * Replaces: ModelRunner.prepare_decode's host loop and copies
 *   (nanovllm/engine/model_runner.py:892-938), the slot formula with
 *   Sequence.last_block_num_tokens (nanovllm/engine/sequence.py:176-183)
 *   and prepare_block_tables (model_runner.py:696-707).
 */
#define NKV_MAX_PACK_SEQS 4096
int nkv_pack_decode(const int32_t* num_tokens, const int32_t* block_offsets,
                    const int32_t* block_ids, int64_t num_block_ids,
                    int64_t num_seqs, int64_t padded_seqs,
                    int64_t block_size, int64_t table_width,
                    int64_t table_stride, int32_t* slot_mapping,
                    int32_t* context_lens, int32_t* block_tables,
                    int32_t* cu_seqlens_k, void* stream);

/*
 * Prefill / chunked-prefill metadata packing on the device.  Per sequence:
 * start = num_cached[i], q = num_scheduled[i], end = start + q.
 *   cu_seqlens_q    [num_seqs+1]  exclusive scan of q
 *   cu_seqlens_k    [num_seqs+1]  exclusive scan of end
 *   slot_mapping    [num_slots]   for every sequence with a non-empty block
 *                                 list, in order, the slots of positions
 *                                 start..end-1:
 *                                 bt[p / block_size]*block_size + p % block_size;
 *                                 sequences with an empty block list emit
 *                                 nothing.  num_slots must equal that total.
 *   block_tables    [num_seqs, table_width] -1 padded (may be NULL)
 *   full_context_lens[i] = num_prompt[i]   (may be NULL with num_prompt)
 *   query_start_lens[i]  = start           (may be NULL)
 *   max_seqlens[0..1]    = max q, max end  (may be NULL)
 *
 * Replaces: ModelRunner.prepare_prefill's metadata part
 *   (nanovllm/engine/model_runner.py:757-820, 856-882).
 */
int nkv_pack_prefill(const int32_t* num_cached, const int32_t* num_scheduled,
                     const int32_t* num_prompt, const int32_t* block_offsets,
                     const int32_t* block_ids, int64_t num_block_ids,
                     int64_t num_seqs,
                     int64_t block_size, int64_t table_width,
                     int64_t num_slots, int32_t* cu_seqlens_q,
                     int32_t* cu_seqlens_k, int32_t* slot_mapping,
                     int32_t* block_tables, int32_t* full_context_lens,
                     int32_t* query_start_lens, int32_t* max_seqlens,
                     void* stream);

/*
 * Paged-attention decode: one query token per sequence attends over its
 * whole context (context_len = cu_seqlens_k[i+1] - cu_seqlens_k[i]) read
 * straight from the paged caches, with no gather.
 *   out[i, h, :] = softmax(scale * q[i, h] . K_i[:, h / G]^T) V_i[:, h / G]
 * for query head h, G = num_q_heads / num_kv_heads (kv head h / G), in fp32
 * with a result in the input type; scale must be finite and positive
 * (NKV_E_INVALID otherwise).  An empty context yields zeros.  dtype
 * NKV_DTYPE_BFLOAT16 or NKV_DTYPE_FLOAT16 (q, caches and out alike),
 * head_dim 128, any num_kv_heads, G <= 16.  The weights are rounded to the
 * input type before the product with V, as flash attention does.
 *
 * Replaces: the decode call flash_attn_with_kvcache(q, k_cache, v_cache,
 *   cache_seqlens=context_lens, block_table=block_tables, softmax_scale,
 *   causal=True) of Attention.forward (nanovllm/layers/attention.py:
 *   122-130); numerically the decode branch of SDPAAttention
 *   (attention.py:284-300: per-request gather, then SDPA with GQA).
 *
 * nkv_build_attention_plan splits the contexts for the decode kernels and
 *   writes the split into `plan` (capacity >= nkv_attention_plan_capacity(
 *   total context tokens, num_seqs, block_size) int4 entries, 16-byte
 *   aligned) and each sequence's first partial into first_part
 *   [num_seqs+1].  Below 8 kv heads (the range split) it lays the contexts
 *   end to end in 16-row chunks and cuts them into equal contiguous ranges,
 *   one per worker (1024 / num_kv_heads per kv head, so that a launch is
 *   one wavefront per SIMD of MI355X; a range crosses sequence
 *   boundaries); from 8 kv heads on (the entry split) it cuts every context
 *   into entries of nkv_attention_entry_rows(block_size) rows (whole
 *   blocks, 768 rows by default), one int4 {row0, rows, seq, 0} each.  It
 *   reads only cu_seqlens_k, so one plan serves every layer of a step; it
 *   is valid for those context lengths and that kv-head count only (a
 *   range plan used with another batch size or kv-head count computes no
 *   partial, and the merge writes NaN to every output; a plan for other
 *   lengths of the same batch computes over the wrong rows).
 * nkv_paged_attention_decode runs the split-K partial kernel (one
 *   wavefront per worker and kv head, or one workgroup per entry and kv
 *   head) and the merge; block_tables
 *   [num_seqs, table_stride] (int32, -1 padded) map context rows to cache
 *   blocks, a block id outside [0, num_blocks) or a row past the table
 *   drops its rows; workspace holds nkv_attention_workspace_bytes(capacity,
 *   num_q_heads, head_dim) bytes (16-byte aligned).  q is [num_seqs,
 *   num_q_heads, head_dim] with row stride q_seq_stride elements; out is
 *   [num_seqs, num_q_heads, head_dim] with row stride out_seq_stride (even).
 */
int64_t nkv_attention_entry_rows(int64_t block_size);
int64_t nkv_attention_plan_capacity(int64_t total_tokens, int64_t num_seqs,
                                    int64_t block_size);
int64_t nkv_attention_workspace_bytes(int64_t capacity, int64_t num_q_heads,
                                      int64_t head_dim);
int nkv_build_attention_plan(const int32_t* cu_seqlens_k, int64_t num_seqs,
                             int64_t block_size, int64_t num_kv_heads,
                             void* plan, int64_t capacity,
                             int32_t* first_part, void* stream);
int nkv_paged_attention_decode(const void* q, int64_t q_seq_stride,
                               const void* key_cache, const void* value_cache,
                               const int32_t* block_tables, int64_t table_stride,
                               const void* plan, int64_t capacity,
                               const int32_t* first_part, int64_t num_seqs,
                               int64_t num_kv_heads, int64_t num_q_heads,
                               int64_t head_dim, int64_t block_size,
                               int64_t num_blocks, float scale, int32_t dtype,
                               void* workspace, int64_t workspace_bytes,
                               void* out, int64_t out_seq_stride, void* stream);

/*
 * Paged-attention prefill: causal attention of each sequence's chunk of
 * query tokens over its context, read straight from the paged cache
 * (head_dim 128, bfloat16 or float16 for q, caches and out alike, query
 * heads per kv head G = 1 to 8).
 * Request i has query rows [cu_seqlens_q[i], cu_seqlens_q[i+1]) (Lq) and
 * context rows [0, Lk), Lk = cu_seqlens_k[i+1] - cu_seqlens_k[i] >= Lq;
 * query j sees keys [0, Lk - Lq + j]; query head h reads kv head h / G.
 *
 * Replaces: the prefill call flash_attn_varlen_func(q, k_cache, v_cache,
 *   cu_seqlens_q, cu_seqlens_k, ..., causal=True, block_table=...) of
 *   Attention.forward (nanovllm/layers/attention.py:95-116); numerics of
 *   SDPAAttention's prefill (attention.py:226-282: per-request gather, then
 *   SDPA with the prefix-causal mask of :155-161).
 *
 * nkv_build_prefill_plan cuts every request's queries into tiles of
 *   nkv_prefill_tile_tokens(G) tokens (128 / G) and writes one int4
 *   {seq, token0, tokens, 0} per tile into `plan` (capacity >=
 *   nkv_prefill_plan_capacity(total query tokens, num_seqs, G)).  Tiles
 *   are listed by the number of keys they see, most first (plans of up to
 *   2048 entries; longer ones request by request, last tile first).  It
 *   reads only cu_seqlens_q and cu_seqlens_k, so one plan serves every
 *   layer of a step.
 * nkv_paged_attention_prefill runs one workgroup per (tile, kv head);
 *   block_tables [num_seqs, table_stride] (int32, -1 padded); a block id
 *   outside [0, num_blocks) or a row past the table drops its keys.  q and
 *   out are [total query tokens, num_q_heads, head_dim] with token strides
 *   q_token_stride / out_token_stride elements (q rows 16-byte aligned,
 *   out rows 8-byte aligned).  Needs no workspace.
 */
int64_t nkv_prefill_tile_tokens(int64_t group);
int64_t nkv_prefill_plan_capacity(int64_t total_q_tokens, int64_t num_seqs,
                                  int64_t group);
int nkv_build_prefill_plan(const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, int64_t num_seqs,
                           int64_t group, void* plan, int64_t capacity,
                           void* stream);
int nkv_paged_attention_prefill(const void* q, int64_t q_token_stride,
                                const void* key_cache, const void* value_cache,
                                const int32_t* block_tables, int64_t table_stride,
                                const int32_t* cu_seqlens_q,
                                const int32_t* cu_seqlens_k, const void* plan,
                                int64_t capacity, int64_t num_seqs,
                                int64_t num_kv_heads, int64_t num_q_heads,
                                int64_t head_dim, int64_t block_size,
                                int64_t num_blocks, float scale, int32_t dtype,
                                void* out, int64_t out_token_stride, void* stream);

/*
 * Host-to-device transfer lane: a non-blocking transfer stream (default
 * priority) and recycled events owned by the library.
 *   nkv_transfer_h2d   copies `bytes` from pinned host `src` to device `dst`
 *                      on the lane, ordered after all work already enqueued
 *                      on `compute_stream`, and makes `compute_stream` wait
 *                      for the copy; returns an increasing ticket.  The host
 *                      buffer must stay valid until the ticket completes.
 *   nkv_transfer_poll  in_flight = copies not yet complete; completed_upto =
 *                      highest completed ticket (copies complete in order).
 *   nkv_transfer_synchronize waits for every copy; destroy synchronizes too.
 *
 * Replaces: the transfer stream, reuse/transfer events and pending-copy
 *   bookkeeping of PagedKVCache::copy_slots_async
 *   (csrc/paged_kv/paged_kv.cpp:67-72, 101-168); the reference's grown slot
 *   buffer and host-tensor retention live with the caller (the Python
 *   owner nanokv.paged_kv.owner.HIPPagedKVCache).
 */
typedef struct nkv_transfer nkv_transfer;
int nkv_transfer_create(int32_t device, nkv_transfer** out);
int nkv_transfer_destroy(nkv_transfer* lane);
int nkv_transfer_h2d(nkv_transfer* lane, void* dst, const void* src,
                     int64_t bytes, void* compute_stream, int64_t* ticket);
int nkv_transfer_poll(nkv_transfer* lane, int64_t* in_flight,
                      int64_t* completed_upto);
int nkv_transfer_synchronize(nkv_transfer* lane);

/*
 * Device block pool: the block bookkeeping of the reference BlockManager,
 * resident in HBM.
 *   - the free-block FIFO: fresh blocks from the front, freed blocks to the
 *     back, a prefix hit on a free block leaving the queue where it stands;
 *   - the reference counts;
 *   - one block table per sequence slot.
 *
 * Replaces: BlockManager._allocate_block / _deallocate_block / allocate /
 *   deallocate / may_append (nanovllm/engine/block_manager.py:87-118,
 *   185-236), and the upload of every sequence's block list that
 *   ModelRunner.prepare_block_tables feeds on (model_runner.py:696-707).
 *   The prefix-hash chain (compute_hash, hash_to_block_id, hash_blocks,
 *   :65-85, 229-258) stays with the caller, which passes each allocation's
 *   cached-prefix block ids.
 *
 * The state lives in one device buffer the caller owns (the library never
 *   allocates): nkv_pool_bytes gives its size, nkv_pool_offsets the byte
 *   offsets of its arrays (META, RING, QPOS, REF, TABLES, NBLK), and an
 *   nkv_pool_desc names the buffer (256-byte aligned) and its geometry.
 * nkv_pool_init initialises the state on `stream`: every block free in id
 *   order, every table empty, no error.
 * nkv_pool_apply runs an op log (device memory, int32) in order on one
 *   workgroup:
 *     ops  [num_ops][4] {type, slot, num_blocks, args_offset}, 16-B aligned;
 *     args for ALLOCATE: args[args_offset] = number of cached-prefix ids k,
 *          then the k ids (distinct; each either used, gaining a reference,
 *          or free, leaving the queue).
 *     ALLOCATE   slot takes num_blocks blocks: the k cached ids, then
 *                num_blocks - k blocks from the queue front (slot must hold
 *                no blocks; num_blocks <= max_blocks_per_seq);
 *     DEALLOCATE slot releases its blocks in reversed table order; a block
 *                whose count reaches zero goes to the back of the queue;
 *     APPEND     slot takes one block from the queue front (the reference
 *                calls may_append when len(seq) % block_size == 1);
 *     FENCE      no-op.
 *   Consecutive APPENDs, and consecutive ALLOCATEs without cached ids, run
 *   as one parallel step up to the first repeated slot; the result is the
 *   one-op-at-a-time result.
 *   Every op is validated before it changes anything.  The first invalid op
 *   (bad slot or block, table busy/full, not enough free blocks) is recorded
 *   in meta[3] (its index + 1) and meta[4] (an NKV_POOL_ERR_* code) and
 *   ends the log; later logs are ignored until nkv_pool_init.
 * The arrays (at nkv_pool_offsets[k], in the order of the NKV_POOL_* ids):
 *     META   int64[8] = head, tail, live free blocks, error op + 1, error
 *            code;
 *     RING   int32[2*num_blocks], the queue, -1 tombstones;
 *     QPOS   int64[num_blocks];
 *     REF    int32[num_blocks];
 *     TABLES int32[max_seqs * max_blocks_per_seq], -1 padded;
 *     NBLK   int32[max_seqs].
 *   Free blocks in order are the non-negative RING entries of absolute
 *   positions [head, tail), ring index = position % (2*num_blocks).
 * nkv_pack_decode_pool / nkv_pack_prefill_pool are nkv_pack_decode /
 *   nkv_pack_prefill with sequence i's block list read from the pool's
 *   table of slot seq_slots[i] instead of a host-built CSR.
 */
typedef struct nkv_pool_desc {
  void* memory;               /* nkv_pool_bytes(...) bytes of device memory */
  int64_t num_blocks;
  int64_t max_seqs;           /* sequence slots */
  int64_t max_blocks_per_seq; /* table width */
} nkv_pool_desc;
#define NKV_POOL_OP_ALLOCATE 1
#define NKV_POOL_OP_DEALLOCATE 2
#define NKV_POOL_OP_APPEND 3
#define NKV_POOL_OP_FENCE 4
#define NKV_POOL_META 0
#define NKV_POOL_RING 1
#define NKV_POOL_QPOS 2
#define NKV_POOL_REF 3
#define NKV_POOL_TABLES 4
#define NKV_POOL_NBLK 5
#define NKV_POOL_ERR_BAD_OP 1        /* unknown op type                  */
#define NKV_POOL_ERR_BAD_SLOT 2      /* slot outside [0, max_seqs)       */
#define NKV_POOL_ERR_TABLE_BUSY 3    /* ALLOCATE on a slot holding blocks */
#define NKV_POOL_ERR_TABLE_FULL 4    /* APPEND past max_blocks_per_seq   */
#define NKV_POOL_ERR_NO_FREE 5       /* not enough free blocks           */
#define NKV_POOL_ERR_BAD_BLOCK 6     /* block id out of range / unowned  */
#define NKV_POOL_ERR_BAD_ARGS 7      /* counts or args offset invalid    */
#define NKV_POOL_MAX_BLOCKS (1 << 28)
#define NKV_POOL_MAX_SEQS 65536
int64_t nkv_pool_bytes(int64_t num_blocks, int64_t max_seqs,
                       int64_t max_blocks_per_seq);
int nkv_pool_offsets(int64_t num_blocks, int64_t max_seqs,
                     int64_t max_blocks_per_seq, int64_t* offsets /* [6] */);
int nkv_pool_init(const nkv_pool_desc* pool, void* stream);
int nkv_pool_apply(const nkv_pool_desc* pool, const int32_t* ops, int64_t num_ops,
                   const int32_t* args, int64_t num_args, void* stream);
int nkv_pack_decode_pool(const nkv_pool_desc* pool, const int32_t* num_tokens,
                         const int32_t* seq_slots, int64_t num_seqs,
                         int64_t padded_seqs, int64_t block_size,
                         int64_t table_width, int64_t table_stride,
                         int32_t* slot_mapping, int32_t* context_lens,
                         int32_t* block_tables, int32_t* cu_seqlens_k,
                         void* stream);
int nkv_pack_prefill_pool(const nkv_pool_desc* pool, const int32_t* num_cached,
                          const int32_t* num_scheduled, const int32_t* num_prompt,
                          const int32_t* seq_slots, int64_t num_seqs,
                          int64_t block_size, int64_t table_width,
                          int64_t num_slots, int32_t* cu_seqlens_q,
                          int32_t* cu_seqlens_k, int32_t* slot_mapping,
                          int32_t* block_tables, int32_t* full_context_lens,
                          int32_t* query_start_lens, int32_t* max_seqlens,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NANOKV_H */
