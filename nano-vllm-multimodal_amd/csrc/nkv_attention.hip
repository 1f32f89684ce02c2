// Paged-attention decode: one query token per sequence attends over its
// context straight from the paged KV cache, so the context is read once and
// never gathered.  This is the consumer the reference's decode path calls
// (flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens, block_table,
// softmax_scale, causal=True), nanovllm/layers/attention.py:122-130); its
// numerical reference is SDPAAttention's decode branch
// (attention.py:284-300: gather, then scaled_dot_product_attention with
// enable_gqa, query head j reading kv head j / (Hq / Hkv)).
//
// Split-K ("flash decoding"): every context is cut into pieces, a kernel
// writes one softmax partial per (piece, query head) (reference max m,
// weight sum l, unnormalised output), and a reduce kernel merges the
// partials of each (sequence, query head).  Two splits, chosen by the kv
// head count (the plan and the decode call decide alike):
//   * the range split (Hkv < 8, attn_decode_range_kernel): the contexts,
//     cut into 16-key chunks, are laid end to end and dealt in equal
//     contiguous ranges to 1024 / Hkv workers per kv head, so the launch is
//     exactly one wavefront per SIMD of the chip's 256 CUs (one 4-wave
//     workgroup per CU); every wavefront streams the same number of bytes
//     and they finish together; a range crosses sequence boundaries freely;
//   * the entry split (Hkv >= 8, attn_decode_entry_kernel): one workgroup
//     per (entry of up to 768 rows of one sequence, kv head), two per CU.
// Entries leave the end of a launch to its last few workgroups, each at a
// single workgroup's latency-bound rate: measured on the 256-sequence
// decode step, the slots left idle after the last workgroup started sum to
// about 14 us of the whole chip, a tenth of a 2-kv-head launch (150 us) but
// under 3% of an 8-kv-head one (540 us).  One wavefront per SIMD streams
// somewhat slower than two workgroups per CU, so the range split wins
// with 2 and 4 kv heads and the entry split with 8.
//
// The G = Hq / Hkv query heads of one kv head are the 16 columns of MFMA
// tiles (G <= 16), so a chunk costs the same 13 MFMAs whatever G is (see
// attn_decode_range_kernel).
#include <cmath>
#include <cstdlib>

#include "nkv_common.h"
#include "nkv_mfma.h"

namespace nkv {
namespace {

// Launch-shape knobs (compile-time; the defaults are the measured best on
// MI355X for the 256-sequence decode step).
#ifndef NKV_DEC_WAVES
#define NKV_DEC_WAVES 4  // wavefronts (workers) per workgroup
#endif
#ifndef NKV_DEC_WAVE_SLOTS
#define NKV_DEC_WAVE_SLOTS 1024  // wavefronts per launch: one per SIMD of MI355X's 256 CUs
#endif
#ifndef NKV_DEC_SLOTS
#define NKV_DEC_SLOTS 2  // chunk buffers per wavefront: kDecSlots - 1 chunks in flight
#endif
#ifndef NKV_DEC_SEG_COST
#define NKV_DEC_SEG_COST 1  // chunks' worth of time a worker spends starting a sequence
#endif
#ifndef NKV_DEC_NT_LOADS
#define NKV_DEC_NT_LOADS 1  // stream K/V past the caches (nt)
#endif
#ifndef NKV_DEC_ENTRY_ROWS
#define NKV_DEC_ENTRY_ROWS 768  // entry split: target context rows per workgroup
#endif
#ifndef NKV_DEC_ENTRY_MIN_KV_HEADS
#define NKV_DEC_ENTRY_MIN_KV_HEADS 8  // kv heads from which the entry split runs
#endif
constexpr int kDecWaves = NKV_DEC_WAVES;
constexpr int kDecThreads = kDecWaves * kWave;
constexpr int kDecWorkers = NKV_DEC_WAVE_SLOTS;  // workers per kv head at most (one kv head)
constexpr int kDecSlots = NKV_DEC_SLOTS;
constexpr int kDecSegCost = NKV_DEC_SEG_COST;
constexpr int kHeadDim = 128;
constexpr int kHeadBytes = kHeadDim * 2;       // bf16 / fp16
constexpr int kDecKeys = 16;                   // keys per chunk
constexpr int kDecChunkWords = kDecKeys * 16;  // 16-byte words per K or V chunk
constexpr int kDecCopies = 2 * kDecKeys / 4;   // copy instructions per chunk (K and V)
constexpr int kDecMaxGroup = 16;               // query heads per kv head (MFMA columns)
constexpr int kDecQBufHeads = 8;               // query heads whose q a worker prefetches into LDS
constexpr int kPlanThreads = 1024;
constexpr int kEntryRows = NKV_DEC_ENTRY_ROWS;
constexpr int kMaxEntryBlocks = 64;  // blocks one entry may span
constexpr int kEntryMinKvHeads = NKV_DEC_ENTRY_MIN_KV_HEADS;
static_assert(kDecWaves == 1 || kDecWaves == 2 || kDecWaves == 4 || kDecWaves == 8,
              "NKV_DEC_WAVES must be 1, 2, 4 or 8");
static_assert(kDecWorkers >= 1 && kDecWorkers <= 65536, "NKV_DEC_WAVE_SLOTS must be in [1, 65536]");
static_assert(kDecSlots >= 2 && kDecSlots <= 4, "NKV_DEC_SLOTS must be in [2, 4]");
static_assert(kDecSegCost >= 0 && kDecSegCost <= 64, "NKV_DEC_SEG_COST must be in [0, 64]");
static_assert(kEntryRows >= 1 && kEntryRows <= 4096, "NKV_DEC_ENTRY_ROWS must be in [1, 4096]");

// Which split a layout runs: the range split below 8 kv heads, the entry
// split from 8 on (the plan and the decode call take the same decision).
__host__ __device__ constexpr bool uses_entries(int64_t num_kv_heads) {
  return num_kv_heads >= kEntryMinKvHeads;
}

// Context rows per entry of the entry split: whole blocks up to
// NKV_DEC_ENTRY_ROWS (at most kMaxEntryBlocks of them, at least one), or,
// for blocks larger than that, the largest divisor of the block that fits.
int64_t attention_entry_rows(int64_t block_size) {
  if (block_size <= kEntryRows) {
    int64_t blocks = kEntryRows / block_size;
    if (blocks > kMaxEntryBlocks) blocks = kMaxEntryBlocks;
    return blocks * block_size;
  }
  int64_t rows = kEntryRows;
  while (rows > 1 && block_size % rows != 0) --rows;
  return rows;
}

// The running max is a reference, moved only when a score exceeds it by more
// than this (log2 units): weights stay <= 2^8, far from fp32 overflow, and
// the rescale of the accumulators (divergent across the heads of a wave)
// becomes rare.  The final merge divides by the sum taken against the same
// reference, so the result is the softmax up to rounding.
constexpr float kRescaleLog2 = 8.f;

typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float half_lo(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w & 0xFFFFu)));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(w >> 16)));
}

// fp32 -> bf16, round to nearest even (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// fp32 rounded to nearest even in the element type: bf16 (kHalf false) or
// fp16 (kHalf true).
template <bool kHalf>
__device__ __forceinline__ uint16_t from_f32(float f) {
  if constexpr (kHalf) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  } else {
    return to_bf16(f);
  }
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Max over the 16 lanes of a DPP row, in every lane of the row: swap
// neighbours, swap pairs, mirror the half rows, mirror the row.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  return v;
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a))) |
         (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(b))) << 16);
}

// s_waitcnt vmcnt(n) with the other counters left alone, and a compiler
// barrier for memory (the LDS reads after it must stay after it).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}
__device__ __forceinline__ void wait_lgkmcnt0() {
  asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
}

// One wavefront copies 4 bytes per lane into LDS: lane l's word lands at
// lds_dst + 4 l (global_load_lds_dword, LDS base in M0), counted like the
// 16-byte copies of nkv_mfma.h.
__device__ __forceinline__ void lds_copy4(const int32_t* src, uint32_t lds_dst) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off"
               :
               : "v"(src), "s"(lds_dst)
               : "m0", "memory");
}

// The plan and first_part seen as constant memory: the kernel never writes
// them, and uniform loads from the constant address space become scalar
// loads.  Through generic pointers they would be vector loads (the copies'
// inline asm clobbers memory, so the compiler cannot prove them unchanged),
// and a vector load waited for with vmcnt(0) also waits for the copies in
// flight.
typedef __attribute__((address_space(4))) const int32_t const_i32;

// ------------------------------------------------------- the range plan
//
// The range split's plan, in int4 units (one plan serves every layer of a step: it
// depends on the context lengths only):
//   [0]                     {workers, units, num_seqs, num_kv_heads}
//   [1, 1 + kDecWorkers)    one record per worker {seq, chunk0, end, 0}
//   then int32 lens[num_seqs] and int32 vstart[num_seqs], each padded to a
//   multiple of 4.
// The split runs on a line of "units": sequence i, with n_i = ceil(len_i /
// 16) chunks, takes kDecSegCost + n_i units (none when empty), the first
// kDecSegCost standing for the time a worker spends starting it (its q, its
// first block ids and, at the end, one more partial); its chunk c sits at
// unit vstart[i] + c.  Worker w owns units [w U / W, (w + 1) U / W) with
// W = min(workers_per_head(Hkv), U), and computes the chunks inside them: from chunk
// chunk0 of sequence seq (its first unit's sequence) up to unit `end`.
// first_part[i] is sequence i's first partial; its partials are numbered by
// worker, so worker w writes partial first_part[i] + w - (worker of
// vstart[i]) for each sequence i it touches.
__host__ __device__ constexpr int64_t plan_seq_words(int64_t num_seqs) {
  return (num_seqs + 3) / 4;  // int4s per per-sequence int32 array
}
// Workers of one kv head: the launch's wavefronts shared by the kv heads.
__host__ __device__ constexpr int64_t workers_per_head(int64_t num_kv_heads) {
  return kDecWorkers / num_kv_heads > 0 ? kDecWorkers / num_kv_heads : 1;
}
__host__ __device__ constexpr int64_t plan_int4s(int64_t num_seqs) {
  return 1 + kDecWorkers + 2 * plan_seq_words(num_seqs);
}
// Plan entries to allocate: the plan itself, and (the workspace is sized
// from the same number) every partial: each worker writes one per sequence
// it touches, at most W + num_seqs in all.
constexpr int64_t range_plan_capacity(int64_t num_seqs) { return kDecWorkers + num_seqs + 4; }
static_assert(plan_int4s(0) <= range_plan_capacity(0) && plan_int4s(1) <= range_plan_capacity(1) &&
                  plan_int4s(3) <= range_plan_capacity(3) && plan_int4s(4) <= range_plan_capacity(4),
              "plan capacity must hold the plan");
// The entry split's plan: one int4 per entry, at most one short entry per
// sequence.
int64_t entry_plan_capacity(int64_t total_tokens, int64_t num_seqs, int64_t block_size) {
  const int64_t rows = attention_entry_rows(block_size);
  return (total_tokens + rows - 1) / rows + num_seqs;
}

// One workgroup: the unit offsets of the sequences by an LDS scan, then the
// partial counts (a second pass over the same runs, straight to
// first_part), then one record per worker by binary search.
__global__ __launch_bounds__(kPlanThreads) void attn_range_plan_kernel(
    const int32_t* __restrict__ cu_seqlens, int32_t num_seqs, int32_t num_kv_heads,
    int4* __restrict__ plan, int32_t* __restrict__ first_part) {
  extern __shared__ int32_t s_mem[];
  int32_t* s_unit = s_mem;                // [num_seqs + 1] first unit of each sequence
  int32_t* s_tmp = s_mem + num_seqs + 1;  // [kPlanThreads / 64 + 1]
  lds_exclusive_scan<kPlanThreads>(
      num_seqs,
      [&](int32_t i) {
        const int32_t len = cu_seqlens[i + 1] - cu_seqlens[i];
        return len > 0 ? (len + kDecKeys - 1) / kDecKeys + kDecSegCost : 0;
      },
      s_unit, s_tmp);
  const int64_t units = s_unit[num_seqs];
  const int64_t per_head = workers_per_head(num_kv_heads);
  const int64_t workers = units < per_head ? units : per_head;
  // The worker owning unit v (units > 0): the largest w with w U / W <= v.
  auto worker_of = [&](int64_t v) { return ((v + 1) * workers - 1) / units; };
  auto parts_of = [&](int32_t i) -> int32_t {
    const int32_t u0 = s_unit[i], u1 = s_unit[i + 1];
    if (u1 == u0) return 0;
    return static_cast<int32_t>(worker_of(u1 - 1) - worker_of(u0 + kDecSegCost) + 1);
  };
  int32_t* lens = reinterpret_cast<int32_t*>(plan + 1 + kDecWorkers);
  int32_t* vstart = lens + 4 * plan_seq_words(num_seqs);
  const int32_t per = (num_seqs + kPlanThreads - 1) / kPlanThreads;
  const int32_t begin = min(num_seqs, static_cast<int32_t>(threadIdx.x) * per);
  const int32_t end = min(num_seqs, begin + per);
  int32_t sum = 0;
  for (int32_t i = begin; i < end; ++i) sum += parts_of(i);
  int32_t total = 0;
  int32_t base = block_exclusive_scan<kPlanThreads>(sum, s_tmp, &total);
  for (int32_t i = begin; i < end; ++i) {
    first_part[i] = base;
    base += parts_of(i);
    lens[i] = cu_seqlens[i + 1] - cu_seqlens[i];
    vstart[i] = s_unit[i] + kDecSegCost;
  }
  if (threadIdx.x == 0) {
    first_part[num_seqs] = total;
    plan[0] = make_int4(static_cast<int32_t>(workers), static_cast<int32_t>(units), num_seqs,
                        num_kv_heads);
  }
  for (int32_t w = threadIdx.x; w < kDecWorkers; w += kPlanThreads) {
    int4 record = make_int4(0, 0, 0, 0);
    if (w < workers) {
      const int64_t first = w * units / workers;
      const int32_t s = owner_of(s_unit, num_seqs, static_cast<int32_t>(first));
      const int32_t chunk0 = static_cast<int32_t>(first) - s_unit[s] - kDecSegCost;
      record = make_int4(s, chunk0 > 0 ? chunk0 : 0,
                         static_cast<int32_t>((w + 1) * units / workers), 0);
    }
    plan[1 + w] = record;
  }
}

// ------------------------------------------- the entry split (Hkv >= 8)
//
// One workgroup per (plan entry, kv head): entries of up to
// attention_entry_rows(block_size) rows of one sequence (768 by default).
// Its wavefronts take the entry's 16-key chunks round-robin and run
// independently, each with a private ring of kDecSlots chunk buffers in LDS
// filled by global_load_lds kDecSlots - 1 chunks ahead of the one it
// computes; the waves then merge through LDS and split the stores of the
// query heads.  The entry's cache rows are resolved once through the block
// table into LDS; invalid rows (block id missing or outside the cache, keys
// past the entry) copy cache row 0 into their slots, their scores are
// masked and their V rows zeroed.  With 8 kv heads a launch is more than
// twenty rounds of workgroups at two per CU, the drain of the last entries
// is a small part of it, and two workgroups per CU stream faster than the
// range split's one wavefront per SIMD.

// The entry plan: one int4 {row0, rows, seq, 0} per entry, rows [row0, row0 + rows)
// of sequence seq's context, entries of a sequence consecutive;
// first_part[i] is sequence i's first entry (first_part[num_seqs] = total).
// Every workgroup rescans the per-sequence entry counts in LDS, so one
// launch builds the whole plan.  Entries past the total get rows = 0.
__global__ __launch_bounds__(kPlanThreads) void attn_entry_plan_kernel(
    const int32_t* __restrict__ cu_seqlens, int32_t num_seqs, int32_t entry_rows,
    int4* __restrict__ plan, int64_t capacity, int32_t* __restrict__ first_part) {
  extern __shared__ int32_t s_mem[];
  int32_t* s_first = s_mem;               // [num_seqs + 1]
  int32_t* s_tmp = s_mem + num_seqs + 1;  // [kPlanThreads / 64 + 1]
  lds_exclusive_scan<kPlanThreads>(
      num_seqs,
      [&](int32_t i) {
        const int32_t len = cu_seqlens[i + 1] - cu_seqlens[i];
        return len > 0 ? (len + entry_rows - 1) / entry_rows : 0;
      },
      s_first, s_tmp);
  if (blockIdx.x == 0) {
    for (int32_t i = threadIdx.x; i <= num_seqs; i += kPlanThreads) first_part[i] = s_first[i];
  }
  const int64_t total = s_first[num_seqs];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kPlanThreads;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kPlanThreads + threadIdx.x; e < capacity;
       e += stride) {
    int4 entry = make_int4(0, 0, 0, 0);
    if (e < total) {
      const int32_t i = owner_of(s_first, num_seqs, static_cast<int32_t>(e));
      const int32_t row0 = (static_cast<int32_t>(e) - s_first[i]) * entry_rows;
      const int32_t len = cu_seqlens[i + 1] - cu_seqlens[i];
      entry = make_int4(row0, min(entry_rows, len - row0), i, 0);
    }
    plan[e] = entry;
  }
}

// Cache row of each context row [row0, row0 + nrows) of sequence seq, -1
// where the block id is missing from the table or outside the cache.  The
// table is read once per block, not once per row: the entry's block ids go
// to `blocks` (LDS, at least nrows ints: every block of the entry holds one
// of its rows) in one round of loads, and the rows are expanded from them
// with no further memory access.  A per-row loop of table loads waits for
// each load before the next (768 rows over 256 threads were three loads in
// a row, about 1.5 us each under load).  Ends with `rows` visible to the
// whole workgroup; `blocks` may be reused after it.
template <int NT>
__device__ __forceinline__ void resolve_rows(const int32_t* __restrict__ tables,
                                             int64_t table_stride, int32_t seq, int32_t row0,
                                             int32_t nrows, int32_t block_size,
                                             int32_t num_blocks, int32_t* blocks,
                                             int32_t* rows) {
  const int32_t first = row0 / block_size;
  const int32_t nblk =
      nrows > 0 ? static_cast<int32_t>((static_cast<int64_t>(row0) + nrows - 1) / block_size) -
                      first + 1
                : 0;
  for (int32_t b = threadIdx.x; b < nblk; b += NT) {
    const int64_t logical = static_cast<int64_t>(first) + b;
    int32_t block = -1;
    if (logical < table_stride) {
      block = tables[static_cast<int64_t>(seq) * table_stride + logical];
      if (block < 0 || block >= num_blocks) block = -1;
    }
    blocks[b] = block;
  }
  __syncthreads();  // block ids in LDS
  for (int32_t t = threadIdx.x; t < nrows; t += NT) {
    const int64_t ctx = static_cast<int64_t>(row0) + t;
    const int32_t block = blocks[ctx / block_size - first];
    rows[t] = block >= 0 ? block * block_size + static_cast<int32_t>(ctx % block_size) : -1;
  }
  __syncthreads();  // rows resolved
}

// Stores one (entry, query head) partial: the wave's lanes hold dims
// 2 lane, 2 lane + 1 of the unnormalised output (a0, a1) against reference
// max mm with weight sum lsum.  The sums go out as fp16 pairs scaled by
// 2^-k, k putting the largest magnitude in [2^14, 2^15); (mm + k, lsum 2^-k)
// carries the same factor, so the merge stays exact.
__device__ __forceinline__ void emit_partial(uint32_t* acc_out, f32x2* ml_out, float a0, float a1,
                                             float mm, float lsum, int lane) {
  // Largest magnitude of the head, in every lane: DPP within rows, then the
  // cross-row swaps (VALU only, no LDS round trips).
  const float amax = row4_max(row16_max(fmaxf(fabsf(a0), fabsf(a1))));
  const int e = static_cast<int>((__float_as_uint(amax) >> 23) & 0xFFu) - 127;
  const int k = amax > 0.f ? min(112, max(-112, e - 14)) : 0;
  const float down = __uint_as_float(static_cast<uint32_t>(127 - k) << 23);
  const uint32_t packed =
      static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a0 * down))) |
      (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a1 * down)))
       << 16);
  store_stream(acc_out + lane, packed);
  if (lane == 0) store_stream(ml_out, f32x2{mm + static_cast<float>(k), lsum * down});
}

// One wavefront's LDS: its ring while it runs, its partials afterwards.
union EntryWaveMem {
  struct {
    u32x4 k[kDecSlots][kDecChunkWords];
    u32x4 v[kDecSlots][kDecChunkWords];
  } ring;
  struct {
    float acc[kDecMaxGroup][kHeadDim];
    float m[kDecMaxGroup];
    float l[kDecMaxGroup];
  } part;
};
struct EntryShared {
  EntryWaveMem wave[kDecWaves];
  int32_t rows[(kEntryRows + kDecKeys - 1) / kDecKeys * kDecKeys];  // whole chunks
};

template <bool kWide, bool kHalf>
__global__ __launch_bounds__(kDecThreads) void attn_decode_entry_kernel(
    const uint16_t* __restrict__ q, int64_t q_seq_stride,
    const uint8_t* __restrict__ key_cache, const uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ tables, int64_t table_stride, int32_t block_size,
    int32_t num_blocks, int32_t num_kv_heads, int32_t group, const int4* __restrict__ plan,
    int32_t num_seqs, float scale_log2, uint32_t* __restrict__ part_acc,
    f32x2* __restrict__ part_ml) {
  typedef Elem<kHalf> E;
  typedef typename E::T T;
  typedef typename E::X8 X8;
  typedef typename E::X4 X4;
  __shared__ EntryShared sh;

  // The kv head rotates with the entry.  Workgroups are dealt to the 8 XCDs
  // round-robin (blockIdx % 8), so head blockIdx % Hkv would pin each XCD to
  // one byte offset inside every cache row; some offsets stream slower than
  // others on MI355X, and the XCD pinned to the slowest ends the launch late
  // (8 kv heads x G = 4: XCDs done after 504-601 us pinned, 556-567 us
  // rotated).  Workgroups of one XCD with the same blockIdx % Hkv are
  // `period` entries apart, so adding part / period walks them over every
  // head; for a fixed entry the heads stay a permutation.
  const int64_t part = blockIdx.x / num_kv_heads;
  const int32_t period = 8 / min(8, num_kv_heads & -num_kv_heads);  // 8 / gcd(Hkv, 8)
  const int32_t kh =
      static_cast<int32_t>((blockIdx.x % num_kv_heads + part / period) % num_kv_heads);
  const int4 entry = plan[part];
  const int32_t row0 = entry.x;
  const int32_t seq = entry.z;
  // Uniform exits for entries outside every sequence; an empty cache
  // (num_blocks == 0) has no row to read, and its entries store (-inf, 0).
  if (entry.y <= 0 || seq < 0 || seq >= num_seqs || row0 < 0) return;
  const int32_t nrows = num_blocks > 0 ? min(entry.y, kEntryRows) : 0;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int c16 = lane & 15;
  const int g4 = lane >> 4;

  // Q^T operands (B of S^T = K Q^T): lane holds head c16 of this kv head,
  // dims 32 dc + 8 g4 .. +8; zero for padding columns.  Loaded first, so
  // they overlap the block-id loads of the rows.
  X8 qb[4];
  {
    const bool col_ok = c16 < group;
    const uint16_t* qrow = q + static_cast<int64_t>(seq) * q_seq_stride +
                           static_cast<int64_t>(kh * group + (col_ok ? c16 : 0)) * kHeadDim;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (col_ok) v = *reinterpret_cast<const u32x4*>(qrow + 32 * dc + 8 * g4);
      qb[dc] = __builtin_bit_cast(X8, v);
    }
  }
  // The block ids pass through wave 0's ring, which no copy fills before
  // the rows are resolved.
  static_assert(sizeof(sh.wave[0].ring) >= kEntryRows * sizeof(int32_t),
                "block-id scratch too small");
  resolve_rows<kDecThreads>(tables, table_stride, seq, row0, nrows, block_size, num_blocks,
                            reinterpret_cast<int32_t*>(&sh.wave[0].ring), sh.rows);
  __builtin_amdgcn_s_waitcnt(0);  // q has landed: only the chunk copies are in flight below

  const uint32_t row_bytes = static_cast<uint32_t>(num_kv_heads) * kHeadBytes;
  const uint8_t* const k_head = key_cache + static_cast<int64_t>(kh) * kHeadBytes;
  const uint8_t* const v_head = value_cache + static_cast<int64_t>(kh) * kHeadBytes;
  EntryWaveMem& mine = sh.wave[wave];
  // LDS byte addresses of this wave's ring (uniform; the copies' M0 base).
  const uint32_t ring_k = lds_address(&sh.wave[0].ring.k[0][0]) +
                          static_cast<uint32_t>(wave) * sizeof(EntryWaveMem);
  const uint32_t ring_v = ring_k + kDecSlots * kDecChunkWords * 16;

  const int32_t nchunks = (nrows + kDecKeys - 1) / kDecKeys;
  const int32_t count = wave < nchunks ? (nchunks - wave + kDecWaves - 1) / kDecWaves : 0;

  // Copies of the wave's chunk j (entry keys 16 (wave + waves j) ..) into
  // slot j % kDecSlots: instruction i moves keys 4 i .. 4 i + 3, lane l the
  // 16-byte chunk that the swizzle puts at position l % 16 of key 4 i + l / 16.
  auto issue = [&](int32_t j) {
    const int32_t key0 = (wave + kDecWaves * j) * kDecKeys;
    const uint32_t slot_off = static_cast<uint32_t>(j % kDecSlots) * kDecChunkWords * 16;
    int32_t row[kDecKeys / 4];
#pragma unroll
    for (int i = 0; i < kDecKeys / 4; ++i) {
      // Read unconditionally (the array holds whole chunks), so the four
      // reads issue together; entries past nrows are never resolved.
      const int32_t t = key0 + 4 * i + g4;
      const int32_t r = sh.rows[t];
      row[i] = t < nrows && r >= 0 ? r : 0;  // invalid: an in-bounds row, masked and zeroed later
    }
#pragma unroll
    for (int i = 0; i < kDecKeys / 4; ++i) {
      const int key = 4 * i + g4;
      const uint32_t kc = 16u * static_cast<uint32_t>(c16 ^ (key & 15));
      const uint32_t vc = 16u * static_cast<uint32_t>(c16 ^ ((key & 7) << 1));
      const uint32_t dst = slot_off + static_cast<uint32_t>(4 * i) * 256u;
      constexpr bool kNt = NKV_DEC_NT_LOADS != 0;
      if (kWide) {
        const int64_t base = static_cast<int64_t>(row[i]) * row_bytes;
        lds_copy16<kNt>(k_head + base + kc, ring_k + dst);
        lds_copy16<kNt>(v_head + base + vc, ring_v + dst);
      } else {
        const uint32_t base = static_cast<uint32_t>(row[i]) * row_bytes;
        lds_copy16<kNt>(k_head, base + kc, ring_k + dst);
        lds_copy16<kNt>(v_head, base + vc, ring_v + dst);
      }
    }
  };

  float row_max = -INFINITY;  // reference max of head c16 (log2 units)
  // O^T blocks: dims 16 db + 4 g4 + i of head c16; block 8 is the ones
  // product, whose g4 == 0, i == 0 entry is the head's weight sum.
  f32x4 acc[9];
#pragma unroll
  for (int db = 0; db < 9; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
  const T one = c16 == 0 ? static_cast<T>(1.f) : static_cast<T>(0.f);
  const X4 ones = {one, one, one, one};
  const int tr_key = 4 * g4 + ((lane >> 2) & 3);  // key this lane addresses in a V^T read
  const int tr_dim = 4 * (lane & 3);              // first dim it addresses, within 16

#pragma unroll
  for (int32_t j = 0; j < kDecSlots - 1; ++j) {
    if (j < count) issue(j);
  }
  for (int32_t j = 0; j < count; ++j) {
    const int32_t ahead = j + kDecSlots - 1;
    if (ahead < count) {
      // The slot receiving chunk `ahead` was read by the previous chunk's
      // products; their LDS reads are complete before it is overwritten.
      asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
      issue(ahead);
    }
    // Chunks issued after j: min(kDecSlots - 1, count - 1 - j), 8 copies each.
    const int32_t later = min(kDecSlots - 1, count - 1 - j);
    if (later >= 3) {
      wait_vmcnt<3 * kDecCopies>();
    } else if (later == 2) {
      wait_vmcnt<2 * kDecCopies>();
    } else if (later == 1) {
      wait_vmcnt<kDecCopies>();
    } else {
      wait_vmcnt<0>();
    }
    const int slot = j % kDecSlots;
    const u32x4* const k_tile = mine.ring.k[slot];
    u32x4* const v_tile = mine.ring.v[slot];
    const int32_t key0 = (wave + kDecWaves * j) * kDecKeys;

    // Keys of this lane's scores (4 g4 + i) and whether each is valid.
    bool bad[4];
    {
      const int32_t t = key0 + 4 * g4;
      const int4 r = *reinterpret_cast<const int4*>(&sh.rows[t]);  // t % 4 == 0, whole chunks
      const int32_t rr[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) bad[i] = t + i >= nrows || rr[i] < 0;
    }
    const bool any_bad = __any(bad[0] || bad[1] || bad[2] || bad[3]);
    if (any_bad) {  // zero V of invalid keys: lane covers key 4 i + g4, chunk c16
#pragma unroll
      for (int i = 0; i < kDecKeys / 4; ++i) {
        const int32_t t = key0 + 4 * i + g4;
        const int32_t r = sh.rows[t];  // whole chunks: in the array
        if (t >= nrows || r < 0) v_tile[(4 * i + g4) * 16 + c16] = u32x4{0u, 0u, 0u, 0u};
      }
    }

    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      const X8 a = __builtin_bit_cast(X8, k_tile[k_index(c16, 4 * dc + g4)]);
      s = E::mfma(a, qb[dc], s);
    }
    if (any_bad) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = bad[i] ? -INFINITY : s[i];
    }
    float local = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    local = row4_max(local) * scale_log2;  // scale > 0: the max commutes with it
    const bool move = local > row_max + kRescaleLog2;
    if (__any(move)) {
      const float m_new = move ? local : row_max;
      const float alpha = move ? exp2_fast(row_max - m_new) : 1.f;  // 0 from -inf
#pragma unroll
      for (int db = 0; db < 9; ++db) acc[db] *= alpha;
      row_max = m_new;
    }
    const float ref = row_max == -INFINITY ? INFINITY : row_max;  // nothing valid yet: weights 0
    X4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = static_cast<T>(exp2_fast(__builtin_fmaf(s[i], scale_log2, -ref)));
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const X4 a = __builtin_bit_cast(X4, v_tr_read(v_tile, tr_key, 16 * db + tr_dim));
      acc[db] = E::mfma16(a, pb, acc[db]);
    }
    acc[8] = E::mfma16(ones, pb, acc[8]);
  }

  // Publish this wave's partials in its own (drained) ring.
  if (c16 < group) {
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      *reinterpret_cast<f32x4*>(&mine.part.acc[c16][16 * db + 4 * g4]) = acc[db];
    }
    if (g4 == 0) {
      mine.part.m[c16] = row_max;
      mine.part.l[c16] = acc[8][0];
    }
  }
  const int64_t num_q_heads = static_cast<int64_t>(num_kv_heads) * group;
  __syncthreads();  // every wave's partials are in LDS
  for (int g = wave; g < group; g += kDecWaves) {
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) mm = fmaxf(mm, sh.wave[w].part.m[g]);
    float a0 = 0.f, a1 = 0.f, lsum = 0.f;
    if (mm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kDecWaves; ++w) {
        const float mw = sh.wave[w].part.m[g];
        const float f = mw == -INFINITY ? 0.f : exp2_fast(mw - mm);
        a0 = fmaf(sh.wave[w].part.acc[g][2 * lane], f, a0);
        a1 = fmaf(sh.wave[w].part.acc[g][2 * lane + 1], f, a1);
        lsum = fmaf(sh.wave[w].part.l[g], f, lsum);
      }
    }
    const int64_t qh = static_cast<int64_t>(kh) * group + g;
    emit_partial(part_acc + (part * num_q_heads + qh) * (kHeadDim / 2),
                 part_ml + part * num_q_heads + qh, a0, a1, mm, lsum, lane);
  }
}

// ------------------------------------------- the range split (Hkv < 8)
//
// Grouped-query decode on MFMA.  The G query heads of one kv head form the
// 16 columns of one MFMA tile (up to 16 heads, padding columns zero), so the
// arithmetic of a 16-key chunk is a fixed 13 MFMAs whatever G is:
//   * S^T = K Q^T: 4 x 16x16x32 (keys x heads, over 128 dims); a lane holds
//     head c16 and keys 4 g4 + i, which is exactly the B layout of a
//     16x16x16 MFMA over those keys, so P^T needs no shuffle;
//   * O^T += V^T P^T: 8 x 16x16x16 (dims x heads, over 16 keys), V^T from
//     the transposing LDS read; a ninth product against a row of ones sums
//     the same (rounded) weights;
//   * the online softmax is a 4-lane max per head and one exp2 per score.
//
// Each wavefront is one worker of the plan, for one kv head, and runs alone
// (no barrier anywhere): a ring of two chunk buffers in LDS, filled by
// global_load_lds one chunk ahead of the chunk it computes and waited for
// with a counted s_waitcnt (8 copies per chunk).  Two walkers follow the
// worker's range: the copy walker one chunk ahead, the compute walker
// behind it.  What a new sequence needs is fetched into LDS, by the same
// kind of copy, before its first chunk's copies, so the count that waits
// for the chunk covers it too:
//   * its first 64 block ids (one per lane), when the copy walker enters the
//     sequence before it; a chunk past those 64 blocks reloads them;
//   * its q (G <= kDecQBufHeads), when the compute walker enters the
//     sequence before it; larger G loads q when the sequence starts.
// A chunk's 16 keys resolve their cache rows through those ids; keys past
// the context or in a block missing from the table or outside the cache
// copy cache row 0 instead and are masked (score -inf, V row zeroed).
//
// When a sequence ends inside the range (or the range ends) the wave writes
// that sequence's partial straight from the MFMA layout: per head, the fp16
// sums of p v 2^-k with k putting the head's largest magnitude in
// [2^14, 2^15) (a 12-bit mantissa for every value well above 2^-27 of the
// largest, no fp16 overflow), and (m + k, l 2^-k); folding k into both
// keeps the merge exact.  A sequence without valid rows gives (-inf, 0).

// One wavefront's LDS.
struct RangeWaveMem {
  u32x4 k[kDecSlots][kDecChunkWords];
  u32x4 v[kDecSlots][kDecChunkWords];
  u32x4 q[kDecQBufHeads * (kHeadBytes / 16)];  // the next sequence's q
  int32_t ids[kWave];                          // the next sequence's first block ids
};

template <bool kWide, bool kHalf>
__global__ __launch_bounds__(kDecThreads) void attn_decode_range_kernel(
    const uint16_t* __restrict__ q, int64_t q_seq_stride,
    const uint8_t* __restrict__ key_cache, const uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ tables, int64_t table_stride, int32_t block_size,
    int32_t num_blocks, int32_t num_kv_heads, int32_t group, const int4* __restrict__ plan_in,
    const int32_t* __restrict__ first_part_in, int32_t num_seqs, int32_t capacity,
    float scale_log2, uint32_t* __restrict__ part_acc, f32x2* __restrict__ part_ml) {
  const const_i32* const plan = (const const_i32*)plan_in;  // int4 entries as int32 words
  const const_i32* const first_part = (const const_i32*)first_part_in;
  typedef Elem<kHalf> E;
  typedef typename E::T T;
  typedef typename E::X8 X8;
  typedef typename E::X4 X4;
  __shared__ RangeWaveMem sh[kDecWaves];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int c16 = lane & 15;
  const int g4 = lane >> 4;

  // Worker w of kv head kh.  Workgroups are dealt to the 8 XCDs round-robin
  // (blockIdx % 8), so a fixed head per wave slot would pin XCDs to byte
  // offsets inside the cache rows, and some offsets stream slower than
  // others on MI355X.  Wavefronts of one XCD with the same worker-relative
  // slot r are `period` workers apart; adding w / period walks them over
  // every head, and for a fixed worker the heads stay a permutation of r.
  const int32_t gw = static_cast<int32_t>(blockIdx.x) * kDecWaves + wave;
  const int32_t w = gw / num_kv_heads;
  const int32_t num_workers = plan[0];
  // An idle worker (fewer units than workers), or a plan built for another
  // batch: nothing is read or written (a plan must come from the same
  // lengths; the partials it would index are not there).
  if (w >= num_workers || num_workers > kDecWorkers || plan[2] != num_seqs ||
      plan[3] != num_kv_heads) {
    return;
  }
  const int32_t r = gw - w * num_kv_heads;
  constexpr int32_t kSpan = 8 * kDecWaves;  // wavefronts per round over the XCDs
  const int32_t period = kSpan / min(kSpan, num_kv_heads & -num_kv_heads);
  const int32_t kh = (r + w / period) % num_kv_heads;

  const int64_t workers = num_workers;
  const int64_t units = plan[1];
  const const_i32* const record = plan + 4 * (1 + w);
  const int32_t end = record[2];  // first unit past the range
  const const_i32* const lens = plan + 4 * (1 + kDecWorkers);
  const const_i32* const vstart = lens + 4 * plan_seq_words(num_seqs);
  int32_t is = record[0];  // copy walker: sequence, chunk, length
  int32_t ic = record[1];
  if (is < 0 || is >= num_seqs || ic < 0) return;
  int32_t ilen = lens[is];
  if (ilen <= 0 || vstart[is] + ic >= end) return;  // a range of start-up units only
  // The next sequence with chunks inside the range, or -1.
  auto next_seq = [&](int32_t s) -> int32_t {
    for (++s; s < num_seqs; ++s) {
      if (lens[s] > 0) return vstart[s] < end ? s : -1;
    }
    return -1;
  };

  RangeWaveMem& mine = sh[wave];
  // LDS byte addresses of this wave's buffers (uniform; the copies' M0 base).
  const uint32_t ring_k = lds_address(&sh[0].k[0][0]) + static_cast<uint32_t>(wave) * sizeof(RangeWaveMem);
  const uint32_t ring_v = ring_k + kDecSlots * kDecChunkWords * 16;
  const uint32_t q_lds = ring_v + kDecSlots * kDecChunkWords * 16;
  const uint32_t ids_lds = q_lds + kDecQBufHeads * kHeadBytes;

  const uint32_t row_bytes = static_cast<uint32_t>(num_kv_heads) * kHeadBytes;
  const uint8_t* const k_head = key_cache + static_cast<int64_t>(kh) * kHeadBytes;
  const uint8_t* const v_head = value_cache + static_cast<int64_t>(kh) * kHeadBytes;
  const uint16_t* const q_head = q + static_cast<int64_t>(kh) * group * kHeadDim;
  const bool q_in_lds = group <= kDecQBufHeads;
  const int32_t q_bytes = group * kHeadBytes;
  const int64_t num_q_heads = static_cast<int64_t>(num_kv_heads) * group;

  // Block ids [first, first + 64) of sequence s's table row, one per lane
  // (-1 past the row or outside the cache); plain loads, checked by
  // valid_id once they have landed.
  auto load_ids = [&](int32_t s, int32_t first) -> int32_t {
    const int64_t b = static_cast<int64_t>(first) + lane;
    return b >= 0 && b < table_stride ? tables[static_cast<int64_t>(s) * table_stride + b] : -1;
  };
  auto valid_id = [&](int32_t id) -> int32_t { return id >= 0 && id < num_blocks ? id : -1; };
  // Block ids [0, 64) of sequence s into the wave's id buffer.
  auto prefetch_ids = [&](int32_t s) {
    if (lane < table_stride) lds_copy4(tables + static_cast<int64_t>(s) * table_stride + lane, ids_lds);
  };
  auto read_ids = [&]() -> int32_t {
    const int32_t id = mine.ids[lane];
    return lane < table_stride && id >= 0 && id < num_blocks ? id : -1;
  };
  // Q^T operands (B of S^T = K Q^T): lane holds head c16 of this kv head,
  // dims 32 dc + 8 g4 .. +8; zero for padding columns.
  auto load_q = [&](int32_t s, X8* qb) {
    const bool col_ok = c16 < group;
    const uint16_t* qrow =
        q_head + static_cast<int64_t>(s) * q_seq_stride + static_cast<int64_t>(col_ok ? c16 : 0) * kHeadDim;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (col_ok) v = *reinterpret_cast<const u32x4*>(qrow + 32 * dc + 8 * g4);
      qb[dc] = __builtin_bit_cast(X8, v);
    }
  };
  // q of sequence s (G heads x 256 contiguous bytes) into the wave's q buffer.
  auto prefetch_q = [&](int32_t s) {
    const uint8_t* src = reinterpret_cast<const uint8_t*>(q_head + static_cast<int64_t>(s) * q_seq_stride);
    for (int32_t off = 0; off < q_bytes; off += kWave * 16) {
      if (off + 16 * lane < q_bytes) lds_copy16<false>(src + off + 16 * lane, q_lds + off);
    }
  };
  auto read_q = [&](X8* qb) {
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (c16 < group) v = mine.q[c16 * (kHeadBytes / 16) + 4 * dc + g4];
      qb[dc] = __builtin_bit_cast(X8, v);
    }
  };

  // Copies of the chunk at context rows t0 .. t0 + 15 of a sequence of
  // length len into ring slot `slot`, through the block ids `ids` of blocks
  // [wb, wb + 64).  Instruction i moves keys 4 i .. 4 i + 3, lane l the
  // 16-byte chunk that the swizzle puts at position l % 16 of key
  // 4 i + l / 16.  Returns the chunk's mask of invalid keys (bit = key).
  auto issue = [&](int32_t slot, int32_t t0, int32_t len, int32_t ids, int32_t wb) -> uint32_t {
    const int32_t blk0 = t0 / block_size;
    const int32_t rem0 = t0 - blk0 * block_size;
    uint32_t bad = 0;
    int32_t row[kDecKeys / 4];
    if (block_size % kDecKeys == 0) {
      // Chunks start at multiples of 16 rows, so the chunk lies in one
      // block: one block id for the wave, and its valid keys are a prefix.
      const int32_t id = __builtin_amdgcn_readlane(ids, blk0 - wb);
      const int32_t valid = id >= 0 ? min(kDecKeys, len - t0) : 0;
      bad = valid >= kDecKeys ? 0u : 0xFFFFu & ~((1u << valid) - 1u);
      const int32_t base = id >= 0 ? id * block_size + rem0 : 0;
#pragma unroll
      for (int i = 0; i < kDecKeys / 4; ++i) {
        const int32_t key = 4 * i + g4;
        row[i] = key < valid ? base + key : 0;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kDecKeys / 4; ++i) {
        const int32_t key = 4 * i + g4;
        int32_t blk, off;
        if (block_size >= kDecKeys) {  // the chunk spans at most two blocks
          const int32_t t = rem0 + key;
          const bool over = t >= block_size;
          blk = blk0 + (over ? 1 : 0);
          off = over ? t - block_size : t;
        } else {
          blk = (t0 + key) / block_size;
          off = t0 + key - blk * block_size;
        }
        const int32_t id = __shfl(ids, (blk - wb) & (kWave - 1), kWave);
        const bool ok = t0 + key < len && id >= 0;
        row[i] = ok ? id * block_size + off : 0;
        const uint64_t invalid = __ballot(!ok);  // key 4 i + g4 is lane 16 g4's bit
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bad |= static_cast<uint32_t>((invalid >> (16 * g)) & 1u) << (4 * i + g);
        }
      }
    }
    if (num_blocks > 0) {  // an empty cache has no row to read: every key is masked
      const uint32_t slot_off = static_cast<uint32_t>(slot) * kDecChunkWords * 16;
#pragma unroll
      for (int i = 0; i < kDecKeys / 4; ++i) {
        const int key = 4 * i + g4;
        const uint32_t kc = 16u * static_cast<uint32_t>(c16 ^ (key & 15));
        const uint32_t vc = 16u * static_cast<uint32_t>(c16 ^ ((key & 7) << 1));
        const uint32_t dst = slot_off + static_cast<uint32_t>(4 * i) * 256u;
        constexpr bool kNt = NKV_DEC_NT_LOADS != 0;
        if (kWide) {
          const int64_t base = static_cast<int64_t>(row[i]) * row_bytes;
          lds_copy16<kNt>(k_head + base + kc, ring_k + dst);
          lds_copy16<kNt>(v_head + base + vc, ring_v + dst);
        } else {
          const uint32_t base = static_cast<uint32_t>(row[i]) * row_bytes;
          lds_copy16<kNt>(k_head, base + kc, ring_k + dst);
          lds_copy16<kNt>(v_head, base + vc, ring_v + dst);
        }
      }
    }
    return bad;
  };

  float row_max = -INFINITY;  // reference max of head c16 (log2 units)
  // O^T blocks: dims 16 db + 4 g4 + i of head c16; block 8 is the ones
  // product, whose g4 == 0, i == 0 entry is the head's weight sum.
  f32x4 acc[9];
#pragma unroll
  for (int db = 0; db < 9; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The partial of the compute walker's sequence, from the MFMA layout.
  auto emit = [&](int32_t part) {
    float amax = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(acc[db][i]));
    }
    amax = row4_max(amax);  // over the head's four lanes
    const int e = static_cast<int>((__float_as_uint(amax) >> 23) & 0xFFu) - 127;
    const int k = amax > 0.f ? min(112, max(-112, e - 14)) : 0;
    const float down = __uint_as_float(static_cast<uint32_t>(127 - k) << 23);
    if (c16 < group && part >= 0 && part < capacity) {
      const int64_t pair = static_cast<int64_t>(part) * num_q_heads + static_cast<int64_t>(kh) * group + c16;
      uint32_t* dst = part_acc + pair * (kHeadDim / 2) + 2 * g4;
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        const u32x2 packed = {pack_f16(acc[db][0] * down, acc[db][1] * down),
                              pack_f16(acc[db][2] * down, acc[db][3] * down)};
        store_stream(reinterpret_cast<u32x2*>(dst + 8 * db), packed);
      }
      if (g4 == 0) store_stream(part_ml + pair, f32x2{row_max + static_cast<float>(k), acc[8][0] * down});
    }
  };

  // The copy walker: (is, ic) is the last chunk issued, ilen its sequence's
  // length, ids / iwb its block ids, nseq the sequence after is.  step()
  // moves it to the next chunk of the range (false at the range's end).
  int32_t iwb = (ic * kDecKeys) / block_size;
  int32_t ids = load_ids(is, iwb);
  int32_t nseq = next_seq(is);
  auto step = [&]() -> bool {
    ++ic;
    if (ic * kDecKeys < ilen) {
      if (vstart[is] + ic >= end) return false;
      const int32_t last = (min(ic * kDecKeys + kDecKeys, ilen) - 1) / block_size;
      if (last - iwb >= kWave) {  // past the 64 block ids held: reload (plain loads)
        iwb = (ic * kDecKeys) / block_size;
        ids = valid_id(load_ids(is, iwb));
      }
      return true;
    }
    if (nseq < 0) return false;
    // The id copy of nseq went out before the first chunk of the sequence
    // now ending, so its last chunk's 8 copies all follow it.
    wait_vmcnt<kDecCopies>();
    is = nseq;
    ic = 0;
    ilen = lens[is];
    iwb = 0;
    ids = read_ids();
    wait_lgkmcnt0();  // read before the buffer is refilled
    nseq = next_seq(is);
    if (nseq >= 0) prefetch_ids(nseq);
    return true;
  };

  // Prologue: the first sequence's block ids and q with plain loads (waited
  // for here, before any copy is in flight), the next sequence's prefetches,
  // then the first kDecSlots - 1 chunks' copies.
  X8 qb[4];
  load_q(is, qb);
  int32_t part = first_part[is] +
                 (w - static_cast<int32_t>(((static_cast<int64_t>(vstart[is]) + 1) * workers - 1) / units));
  __builtin_amdgcn_s_waitcnt(0);
  ids = valid_id(ids);
  int32_t cs = is, cc = ic, clen = ilen;  // compute walker: sequence, chunk, length
  bool q_stale = false;  // the compute walker entered a new sequence: qb is read first
  bool q_late = false;   // its q was copied after its first chunk's copies
  if (nseq >= 0) {
    prefetch_ids(nseq);
    if (q_in_lds) prefetch_q(nseq);
  }
  // Masks of the chunks in flight, the one computed next first.
  uint32_t bad[kDecSlots];
#pragma unroll
  for (int k = 0; k < kDecSlots; ++k) bad[k] = 0;
  bad[0] = issue(0, ic * kDecKeys, ilen, ids, iwb);
  int32_t issued = 1;
  bool copying = true;  // the copy walker has chunks left
#pragma unroll
  for (int k = 1; k < kDecSlots - 1; ++k) {
    if (copying && step()) {
      bad[k] = issue(k, ic * kDecKeys, ilen, ids, iwb);
      ++issued;
    } else {
      copying = false;
    }
  }
  int32_t slot = 0;                        // ring slot of the chunk computed next
  int32_t slot_in = issued % kDecSlots;    // ring slot of the chunk issued next

  const T one = c16 == 0 ? static_cast<T>(1.f) : static_cast<T>(0.f);
  const X4 ones = {one, one, one, one};
  const int tr_key = 4 * g4 + ((lane >> 2) & 3);  // key this lane addresses in a V^T read
  const int tr_dim = 4 * (lane & 3);              // first dim it addresses, within 16

  for (int32_t j = 0;; ++j) {
    // The copy walker issues chunk j + kDecSlots - 1 into the slot chunk
    // j - 1 was computed from.
    if (copying && step()) {
      wait_lgkmcnt0();  // the slot's previous chunk has been read
      bad[kDecSlots - 1] = issue(slot_in, ic * kDecKeys, ilen, ids, iwb);
      ++issued;
      slot_in = slot_in == kDecSlots - 1 ? 0 : slot_in + 1;
    } else {
      copying = false;
    }
    // Chunk j's copies (and everything before them) have landed once no
    // more than the later chunks' copies are outstanding.
    const int32_t later = issued - 1 - j;
    if (later >= 3) {
      wait_vmcnt<3 * kDecCopies>();
    } else if (later == 2) {
      wait_vmcnt<2 * kDecCopies>();
    } else if (later == 1) {
      wait_vmcnt<kDecCopies>();
    } else {
      wait_vmcnt<0>();
    }

    if (q_stale) {  // first chunk of the compute walker's sequence
      if (q_in_lds) {
        if (q_late) wait_vmcnt<0>();
        read_q(qb);
        wait_lgkmcnt0();  // read before the buffer is refilled
        const int32_t after = next_seq(cs);
        if (after >= 0) {
          prefetch_q(after);
          q_late = after <= is;  // its first chunk is already in flight
        }
      } else {
        load_q(cs, qb);
        // Waited for here, where the compiler sees it: a load it still
        // counts as pending would have it wait (vmcnt(0)) before every use
        // of qb, on every chunk.
        __builtin_amdgcn_s_waitcnt(0);
      }
      q_stale = false;
    }

    const uint32_t bad_j = bad[0];
    const u32x4* const k_tile = mine.k[slot];
    u32x4* const v_tile = mine.v[slot];
    if (bad_j != 0) {  // zero V of invalid keys: lane covers key 4 i + g4, chunk c16
#pragma unroll
      for (int i = 0; i < kDecKeys / 4; ++i) {
        if ((bad_j >> (4 * i + g4)) & 1u) v_tile[(4 * i + g4) * 16 + c16] = u32x4{0u, 0u, 0u, 0u};
      }
    }
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      const X8 a = __builtin_bit_cast(X8, k_tile[k_index(c16, 4 * dc + g4)]);
      s = E::mfma(a, qb[dc], s);
    }
    if (bad_j != 0) {  // this lane's scores are keys 4 g4 + i
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = (bad_j >> (4 * g4 + i)) & 1u ? -INFINITY : s[i];
    }
    float local = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    local = row4_max(local) * scale_log2;  // scale > 0: the max commutes with it
    const bool move = local > row_max + kRescaleLog2;
    if (__any(move)) {
      const float m_new = move ? local : row_max;
      const float alpha = move ? exp2_fast(row_max - m_new) : 1.f;  // 0 from -inf
#pragma unroll
      for (int db = 0; db < 9; ++db) acc[db] *= alpha;
      row_max = m_new;
    }
    const float ref = row_max == -INFINITY ? INFINITY : row_max;  // nothing valid yet: weights 0
    X4 pb;
#pragma unroll
    for (int i = 0; i < 4; ++i) pb[i] = static_cast<T>(exp2_fast(__builtin_fmaf(s[i], scale_log2, -ref)));
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const X4 a = __builtin_bit_cast(X4, v_tr_read(v_tile, tr_key, 16 * db + tr_dim));
      acc[db] = E::mfma16(a, pb, acc[db]);
    }
    acc[8] = E::mfma16(ones, pb, acc[8]);

    // The compute walker steps to the next chunk: past its sequence's end it
    // writes the sequence's partial, and moves to the next sequence (whose
    // first partial in this range is this worker's: it is that sequence's
    // first worker).
    const bool last = j + 1 == issued;
    ++cc;
    if (last || cc * kDecKeys >= clen) {
      emit(part);
      if (last) break;
      cs = next_seq(cs);
      cc = 0;
      clen = lens[cs];
      part = first_part[cs];
      q_stale = true;
      row_max = -INFINITY;
#pragma unroll
      for (int db = 0; db < 9; ++db) acc[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < kDecSlots - 1; ++k) bad[k] = bad[k + 1];
    slot = slot == kDecSlots - 1 ? 0 : slot + 1;
  }
}

// Merges the partials of (sequence, query head) pairs, one wavefront per
// pair and no LDS or barrier: lane i loads part i's (m + k, l 2^-k), and
// every lane loads its two dims (one fp16 pair) of up to kReduceBatch parts
// in the same round trip, so the merge waits for memory twice (the
// sequence's part range, then the parts) instead of three times.  The wave
// takes the parts' max with lane shuffles, weights and sums the parts in
// fp32 (part i's m and l come from lane i by shuffle) and divides once.  A
// sequence of more than kReduceBatch parts goes in batches, the running sums
// rescaled when a later batch raises the max.
constexpr int kReduceWaves = 4;  // pairs per workgroup
constexpr int kReduceThreads = kReduceWaves * kWave;
constexpr int kReduceBatch = 8;  // parts in flight per lane

template <bool kHalf>
__global__ __launch_bounds__(kReduceThreads) void attn_decode_reduce_kernel(
    const uint32_t* __restrict__ part_acc, const f32x2* __restrict__ part_ml,
    const int32_t* __restrict__ first_part, const int4* __restrict__ range_plan,
    int32_t num_kv_heads, int64_t capacity, int32_t num_seqs, int32_t num_q_heads,
    uint16_t* __restrict__ out, int64_t out_seq_stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * kReduceWaves + wave;
  if (pair >= static_cast<int64_t>(num_seqs) * num_q_heads) return;  // whole waves; no barrier
  const int32_t seq = static_cast<int32_t>(pair / num_q_heads);
  const int32_t qh = static_cast<int32_t>(pair % num_q_heads);
  uint16_t* const dst = out + static_cast<int64_t>(seq) * out_seq_stride + qh * kHeadDim + 2 * lane;
  // A range plan built for another sequence or kv-head count: the range
  // kernel wrote no partial, so the workspace holds stale values.  Every
  // output becomes NaN instead.
  if (range_plan != nullptr) {
    const const_i32* const header = (const const_i32*)range_plan;
    if (header[2] != num_seqs || header[3] != num_kv_heads) {
      const uint16_t nan = kHalf ? 0x7E00u : 0x7FC0u;
      *reinterpret_cast<uint32_t*>(dst) = static_cast<uint32_t>(nan) | (static_cast<uint32_t>(nan) << 16);
      return;
    }
  }
  const int64_t p0 = max(0, first_part[seq]);
  const int64_t p1 = min(capacity, static_cast<int64_t>(first_part[seq + 1]));

  float run_max = -INFINITY;  // max of the parts merged so far
  float ax = 0.f, ay = 0.f, lsum = 0.f;
  for (int64_t b = p0; b < p1; b += kReduceBatch) {
    const int n = static_cast<int>(min(static_cast<int64_t>(kReduceBatch), p1 - b));
    f32x2 ml = {-INFINITY, 0.f};  // lane i < n: part b + i's (m + k, l 2^-k)
    if (lane < n) ml = part_ml[(b + lane) * num_q_heads + qh];
    uint32_t v[kReduceBatch];
#pragma unroll
    for (int i = 0; i < kReduceBatch; ++i) {
      v[i] = i < n ? part_acc[((b + i) * num_q_heads + qh) * (kHeadDim / 2) + lane] : 0u;
    }
    float m = ml.x;
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, kWave));
    const float new_max = fmaxf(run_max, m);
    if (new_max == -INFINITY) continue;  // nothing valid yet (uniform across the wave)
    const float keep = exp2_fast(run_max - new_max);  // 0 while run_max is -inf
    ax *= keep;
    ay *= keep;
    lsum *= keep;
#pragma unroll
    for (int i = 0; i < kReduceBatch; ++i) {
      if (i < n) {
        const float mi = __shfl(ml.x, i, kWave);
        const float li = __shfl(ml.y, i, kWave);
        const float f = mi == -INFINITY ? 0.f : exp2_fast(mi - new_max);
        ax = fmaf(half_lo(v[i]), f, ax);
        ay = fmaf(half_hi(v[i]), f, ay);
        lsum = fmaf(li, f, lsum);
      }
    }
    run_max = new_max;
  }
  const bool any = lsum > 0.f;
  const uint32_t packed = static_cast<uint32_t>(from_f32<kHalf>(any ? ax / lsum : 0.f)) |
                          (static_cast<uint32_t>(from_f32<kHalf>(any ? ay / lsum : 0.f)) << 16);
  *reinterpret_cast<uint32_t*>(dst) = packed;
}

using RangeKernel = void (*)(const uint16_t*, int64_t, const uint8_t*, const uint8_t*,
                              const int32_t*, int64_t, int32_t, int32_t, int32_t, int32_t,
                              const int4*, const int32_t*, int32_t, int32_t, float, uint32_t*,
                              f32x2*);
using EntryKernel = void (*)(const uint16_t*, int64_t, const uint8_t*, const uint8_t*,
                              const int32_t*, int64_t, int32_t, int32_t, int32_t, int32_t,
                              const int4*, int32_t, float, uint32_t*, f32x2*);

RangeKernel range_kernel_for(bool wide, bool half) {
  if (wide) return half ? attn_decode_range_kernel<true, true> : attn_decode_range_kernel<true, false>;
  return half ? attn_decode_range_kernel<false, true> : attn_decode_range_kernel<false, false>;
}
EntryKernel entry_kernel_for(bool wide, bool half) {
  if (wide) return half ? attn_decode_entry_kernel<true, true> : attn_decode_entry_kernel<true, false>;
  return half ? attn_decode_entry_kernel<false, true> : attn_decode_entry_kernel<false, false>;
}

}  // namespace
}  // namespace nkv

extern "C" int64_t nkv_attention_entry_rows(int64_t block_size) {
  return block_size > 0 ? nkv::attention_entry_rows(block_size) : 0;
}

// Entries to allocate for a plan of either split (the larger of the two),
// which also sizes the workspace: every partial has an entry's index.
extern "C" int64_t nkv_attention_plan_capacity(int64_t total_tokens, int64_t num_seqs,
                                               int64_t block_size) {
  if (total_tokens < 0 || num_seqs < 0 || block_size <= 0) return 0;
  const int64_t ranges = nkv::range_plan_capacity(num_seqs);
  const int64_t entries = nkv::entry_plan_capacity(total_tokens, num_seqs, block_size);
  return ranges > entries ? ranges : entries;
}

extern "C" int64_t nkv_attention_workspace_bytes(int64_t capacity, int64_t num_q_heads,
                                                 int64_t head_dim) {
  if (capacity < 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  // per (partial, query head): head_dim fp16 sums and a float2 (m + k, l * 2^-k)
  return capacity * num_q_heads * (head_dim * 2 + 8);
}

extern "C" int nkv_build_attention_plan(const int32_t* cu_seqlens_k, int64_t num_seqs,
                                        int64_t block_size, int64_t num_kv_heads, void* plan,
                                        int64_t capacity, int32_t* first_part, void* stream) {
  using namespace nkv;
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: num_seqs=%lld outside [0, %d]",
                    static_cast<long long>(num_seqs), NKV_MAX_PLAN_SEQS);
  }
  if (block_size <= 0 || block_size > INT32_MAX || capacity < 0 || capacity > INT32_MAX ||
      num_kv_heads <= 0 || num_kv_heads > INT32_MAX / kDecWorkers) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_build_attention_plan: bad block_size, num_kv_heads or capacity");
  }
  const bool entries = uses_entries(num_kv_heads);
  if (!entries && capacity < range_plan_capacity(num_seqs)) {
    return nkv_fail(NKV_E_CAPACITY,
                    "nkv_build_attention_plan: capacity %lld < %lld entries for %lld sequences",
                    static_cast<long long>(capacity),
                    static_cast<long long>(range_plan_capacity(num_seqs)),
                    static_cast<long long>(num_seqs));
  }
  if (!first_part || (num_seqs > 0 && !cu_seqlens_k) || ((capacity > 0 || !entries) && !plan)) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: plan must be 16-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t lds = (static_cast<size_t>(num_seqs) + 1 + kPlanThreads / kWave + 1) *
                     sizeof(int32_t);
  if (entries) {
    // The entry kernel covers only the entries the capacity holds; a plan
    // too short for the lengths is refused by the caller, who knows them.
    const int64_t blocks = capacity > 0 ? (capacity + kPlanThreads - 1) / kPlanThreads : 1;
    attn_entry_plan_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kPlanThreads), lds, s>>>(
        cu_seqlens_k, static_cast<int32_t>(num_seqs),
        static_cast<int32_t>(attention_entry_rows(block_size)), static_cast<int4*>(plan),
        capacity, first_part);
  } else {
    attn_range_plan_kernel<<<dim3(1), dim3(kPlanThreads), lds, s>>>(
        cu_seqlens_k, static_cast<int32_t>(num_seqs), static_cast<int32_t>(num_kv_heads),
        static_cast<int4*>(plan), first_part);
  }
  return nkv_check_launch("nkv_build_attention_plan");
}

extern "C" int nkv_paged_attention_decode(
    const void* q, int64_t q_seq_stride, const void* key_cache, const void* value_cache,
    const int32_t* block_tables, int64_t table_stride, const void* plan, int64_t capacity,
    const int32_t* first_part, int64_t num_seqs, int64_t num_kv_heads, int64_t num_q_heads,
    int64_t head_dim, int64_t block_size, int64_t num_blocks, float scale, int32_t dtype,
    void* workspace, int64_t workspace_bytes, void* out, int64_t out_seq_stride, void* stream) {
  using namespace nkv;
  if (dtype != NKV_DTYPE_BFLOAT16 && dtype != NKV_DTYPE_FLOAT16) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: only bfloat16 and float16 are supported");
  }
  const bool half = dtype == NKV_DTYPE_FLOAT16;
  if (head_dim != kHeadDim) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: head_dim must be %d", kHeadDim);
  }
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: num_q_heads must be a multiple of num_kv_heads");
  }
  const int64_t group = num_q_heads / num_kv_heads;
  if (group > kDecMaxGroup) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: unsupported head layout %lld kv x %lld q "
                    "(at most %d query heads per kv head)",
                    static_cast<long long>(num_kv_heads), static_cast<long long>(num_q_heads),
                    kDecMaxGroup);
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS || capacity < 0 || capacity > INT32_MAX ||
      block_size <= 0 || num_blocks < 0 || num_blocks * block_size > INT32_MAX ||
      table_stride < 0 || q_seq_stride < num_q_heads * head_dim ||
      out_seq_stride < num_q_heads * head_dim || num_kv_heads * head_dim * 2 > INT32_MAX ||
      num_kv_heads > INT32_MAX / kDecWorkers) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: bad sizes or strides");
  }
  // The kernel relies on scale > 0: it takes the chunk max of the raw
  // scores (masked rows at -inf) before scaling, which commutes with a
  // positive scale only (0 or a negative scale would turn masked rows into
  // NaN or +inf weights).
  if (!std::isfinite(scale) || !(scale > 0.f)) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: scale must be finite and positive");
  }
  if (num_seqs == 0) return NKV_OK;
  const bool entries = uses_entries(num_kv_heads);
  if (!entries && capacity < range_plan_capacity(num_seqs)) {
    return nkv_fail(NKV_E_CAPACITY,
                    "nkv_paged_attention_decode: plan capacity %lld < %lld for %lld sequences",
                    static_cast<long long>(capacity),
                    static_cast<long long>(range_plan_capacity(num_seqs)),
                    static_cast<long long>(num_seqs));
  }
  const int64_t need = nkv_attention_workspace_bytes(capacity, num_q_heads, head_dim);
  if (workspace_bytes < need) {
    return nkv_fail(NKV_E_CAPACITY,
                    "nkv_paged_attention_decode: workspace of %lld bytes < %lld needed",
                    static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  }
  if (!q || !key_cache || !value_cache || !first_part || !out ||
      ((capacity > 0 || !entries) && (!plan || !workspace)) ||
      (table_stride > 0 && !block_tables)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: null pointer");
  }
  if ((reinterpret_cast<uint64_t>(q) | reinterpret_cast<uint64_t>(key_cache) |
       reinterpret_cast<uint64_t>(value_cache) | reinterpret_cast<uint64_t>(plan) |
       reinterpret_cast<uint64_t>(workspace) | static_cast<uint64_t>(q_seq_stride * 2)) % 16 != 0 ||
      (reinterpret_cast<uint64_t>(out) | static_cast<uint64_t>(out_seq_stride * 2)) % 4 != 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: q/caches/plan/workspace must be 16-byte aligned "
                    "and out rows 4-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const float scale_log2 = scale * 1.4426950408889634f;  // log2(e)
  auto* part_acc = static_cast<uint32_t*>(workspace);  // fp16 pairs
  auto* part_ml = reinterpret_cast<f32x2*>(part_acc + capacity * num_q_heads * head_dim / 2);
  // byte offsets into a cache past 4 GiB need 64-bit addresses
  const bool wide = num_blocks * block_size * num_kv_heads * head_dim * 2 > UINT32_MAX;
  if (entries && capacity > 0) {
    if (capacity * num_kv_heads > INT32_MAX) {
      return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: plan too long for the grid");
    }
    entry_kernel_for(wide, half)<<<dim3(static_cast<unsigned>(capacity * num_kv_heads)),
                                   dim3(kDecThreads), 0, s>>>(
        static_cast<const uint16_t*>(q), q_seq_stride, static_cast<const uint8_t*>(key_cache),
        static_cast<const uint8_t*>(value_cache), block_tables, table_stride,
        static_cast<int32_t>(block_size), static_cast<int32_t>(num_blocks),
        static_cast<int32_t>(num_kv_heads), static_cast<int32_t>(group),
        static_cast<const int4*>(plan), static_cast<int32_t>(num_seqs), scale_log2, part_acc,
        part_ml);
  } else if (!entries) {
    const int64_t waves = workers_per_head(num_kv_heads) * num_kv_heads;
    range_kernel_for(wide, half)<<<dim3(static_cast<unsigned>((waves + kDecWaves - 1) / kDecWaves)),
                                   dim3(kDecThreads), 0, s>>>(
        static_cast<const uint16_t*>(q), q_seq_stride, static_cast<const uint8_t*>(key_cache),
        static_cast<const uint8_t*>(value_cache), block_tables, table_stride,
        static_cast<int32_t>(block_size), static_cast<int32_t>(num_blocks),
        static_cast<int32_t>(num_kv_heads), static_cast<int32_t>(group),
        static_cast<const int4*>(plan), first_part, static_cast<int32_t>(num_seqs),
        static_cast<int32_t>(capacity), scale_log2, part_acc, part_ml);
  }
  if (int rc = nkv_check_launch("nkv_paged_attention_decode (partials)")) return rc;
  // one wavefront per (sequence, query head) pair, kReduceWaves pairs per workgroup
  const int64_t pairs = num_seqs * num_q_heads;
  const int4* const range_plan = entries ? nullptr : static_cast<const int4*>(plan);
  const dim3 reduce_grid(static_cast<unsigned>((pairs + kReduceWaves - 1) / kReduceWaves));
  if (half) {
    attn_decode_reduce_kernel<true><<<reduce_grid, dim3(kReduceThreads), 0, s>>>(
        part_acc, part_ml, first_part, range_plan, static_cast<int32_t>(num_kv_heads), capacity,
        static_cast<int32_t>(num_seqs), static_cast<int32_t>(num_q_heads),
        static_cast<uint16_t*>(out), out_seq_stride);
  } else {
    attn_decode_reduce_kernel<false><<<reduce_grid, dim3(kReduceThreads), 0, s>>>(
        part_acc, part_ml, first_part, range_plan, static_cast<int32_t>(num_kv_heads), capacity,
        static_cast<int32_t>(num_seqs), static_cast<int32_t>(num_q_heads),
        static_cast<uint16_t*>(out), out_seq_stride);
  }
  return nkv_check_launch("nkv_paged_attention_decode (reduce)");
}
