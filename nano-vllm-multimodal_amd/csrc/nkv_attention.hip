// Paged-attention decode: one query token per sequence attends over its
// context straight from the paged KV cache, so the context is read once and
// never gathered.  This is the consumer the reference's decode path calls
// (flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens, block_table,
// softmax_scale, causal=True), nanovllm/layers/attention.py:122-130); its
// numerical reference is SDPAAttention's decode branch
// (attention.py:284-300: gather, then scaled_dot_product_attention with
// enable_gqa, query head j reading kv head j / (Hq / Hkv)).
//
// Split-K ("flash decoding"): the context of every sequence is cut into
// entries of up to attention_entry_rows(block_size) rows (768 by default,
// whole blocks), one workgroup per entry computes softmax partials (reference
// max m, weight sum l, unnormalised output), and a reduce kernel merges the
// partials of each (sequence, query head).  Two kernels write the partials:
//
// VALU kernel, G = Hq / Hkv = 1 or 2 (Hkv = 1, 2, 4, 8), on request, one
// workgroup per entry for all heads (8 waves):
//   * the entry's cache rows are resolved once through the block table into
//     LDS (invalid block ids give rows that are skipped);
//   * a 16-lane DPP row owns one (row, kv head): each lane holds 8 dims
//     (16 bytes), so a wavefront instruction reads 1 KiB of consecutive
//     cache bytes (coalesced, non-temporal); the waves take interleaved
//     groups of rows, so the workgroup sweeps its rows as one front;
//   * q.k for the G query heads of that kv head is 4 v_dot2 on packed
//     bf16 / fp16 pairs plus a 4-step DPP row sum (fp32);
//   * an online softmax in fp32 with exp2 (scale * log2 e folded in);
//   * the waves merge in LDS: after one barrier each wave merges and stores
//     its share of the query heads (fp16 sums with a power-of-two scale).
// At G <= 2 its VALU work stays under the memory time.
//
// MFMA kernel, G = 1..16 and any kv-head count (the default for every
// layout): one workgroup per (entry, kv head), the G query heads as the
// columns of 16x16 MFMA tiles (see attn_decode_mfma_kernel); the VALU cost
// of 2 G FLOPs per cache byte would outrun the memory time from G = 3 on,
// and with the kv head rotated over the XCDs the MFMA kernel is also the
// faster one at G = 1 and 2.  The VALU kernel runs the G <= 2 layouts it
// covers when NKV_DECODE_VALU=1 is set.
#include <cmath>
#include <cstdlib>

#include "nkv_common.h"
#include "nkv_mfma.h"

namespace nkv {
namespace {

// Launch-shape knobs (compile-time; the defaults are the measured best on
// MI355X for the 256-sequence decode step).
#ifndef NKV_ATTN_WAVES
#define NKV_ATTN_WAVES 8  // wavefronts per workgroup
#endif
#ifndef NKV_ATTN_UNROLL
#define NKV_ATTN_UNROLL 4  // row loads in flight per lane per iteration
#endif
#ifndef NKV_ATTN_ENTRY_ROWS
#define NKV_ATTN_ENTRY_ROWS 768  // target context rows per workgroup
#endif
#ifndef NKV_ATTN_NT_LOADS
#define NKV_ATTN_NT_LOADS 1  // non-temporal K/V loads
#endif
#ifndef NKV_ATTN_WAVES_PER_EU
#define NKV_ATTN_WAVES_PER_EU 0  // >0: ask for that many waves per SIMD (caps VGPRs)
#endif
#if NKV_ATTN_WAVES_PER_EU > 0
#define NKV_ATTN_OCCUPANCY __attribute__((amdgpu_waves_per_eu(NKV_ATTN_WAVES_PER_EU)))
#else
#define NKV_ATTN_OCCUPANCY
#endif

constexpr int kAttnWaves = NKV_ATTN_WAVES;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kHeadDim = 128;
constexpr int kHeadBytes = kHeadDim * 2;  // bf16
constexpr int kAttnUnroll = NKV_ATTN_UNROLL;
constexpr int kMaxQHeads = 16;  // the waves' LDS merge buffer: 4 KiB per query head
constexpr int kEntryRows = NKV_ATTN_ENTRY_ROWS;
constexpr int kMaxEntryBlocks = 64;  // blocks one entry may span
constexpr int kPlanThreads = 1024;
static_assert(kAttnWaves == 1 || kAttnWaves == 2 || kAttnWaves == 4 || kAttnWaves == 8,
              "NKV_ATTN_WAVES must be 1, 2, 4 or 8");
static_assert(kAttnUnroll >= 1 && kAttnUnroll <= 8, "NKV_ATTN_UNROLL must be in [1, 8]");
static_assert(kEntryRows >= 1 && kEntryRows <= 4096, "NKV_ATTN_ENTRY_ROWS must be in [1, 4096]");

// The running max is a reference, moved only when a score exceeds it by more
// than this (log2 units): weights stay <= 2^8, far from fp32 overflow, and
// the rescale of the accumulators (divergent across the heads of a wave)
// becomes rare.  The final merge divides by the sum taken against the same
// reference, so the result is the softmax up to rounding.
constexpr float kRescaleLog2 = 8.f;

// Context rows per plan entry: whole blocks up to NKV_ATTN_ENTRY_ROWS (at
// most kMaxEntryBlocks of them, at least one), or, for blocks larger than
// that, the largest divisor of the block that fits.
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

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// One v_dot2 on a packed bf16 pair.  The words arrive as scalars on purpose:
// __builtin_bit_cast applied directly to an ext_vector component (a.y) is
// lowered by this clang to component 0 for every component.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a),
                                         __builtin_bit_cast(bf16x2v, b), acc, false);
}

typedef _Float16 f16x2v __attribute__((ext_vector_type(2)));
// The same on a packed fp16 pair (v_dot2_f32_f16).
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2v, a), __builtin_bit_cast(f16x2v, b), acc,
                                false);
}

// Dot product of 8 packed elements: bf16 (kHalf false) or fp16 (kHalf true).
template <bool kHalf>
__device__ __forceinline__ float dot8(u32x4 a, u32x4 b, float acc) {
  if constexpr (kHalf) {
    acc = dot2_f16(a.x, b.x, acc);
    acc = dot2_f16(a.y, b.y, acc);
    acc = dot2_f16(a.z, b.z, acc);
    return dot2_f16(a.w, b.w, acc);
  } else {
    acc = dot2_bf16(a.x, b.x, acc);
    acc = dot2_bf16(a.y, b.y, acc);
    acc = dot2_bf16(a.z, b.z, acc);
    return dot2_bf16(a.w, b.w, acc);
  }
}

// Sum over the 16 lanes of a DPP row: swap neighbours, swap pairs, mirror
// the half rows, mirror the row.  Every lane of the row ends with the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
  v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
  return v;
}

// Max over the 16 lanes of a DPP row, in every lane of the row (the same
// four steps as row16_sum).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  return v;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

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

// Element <-> fp32 for the two 16-bit types: the low / high half of a word,
// and fp32 rounded to nearest even.
template <bool kHalf>
__device__ __forceinline__ float elem_lo(uint32_t w) { return kHalf ? half_lo(w) : bf16_lo(w); }
template <bool kHalf>
__device__ __forceinline__ float elem_hi(uint32_t w) { return kHalf ? half_hi(w) : bf16_hi(w); }
template <bool kHalf>
__device__ __forceinline__ uint16_t from_f32(float f) {
  if constexpr (kHalf) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
  } else {
    return to_bf16(f);
  }
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Plan: one int4 {row0, rows, seq, 0} per entry, rows [row0, row0 + rows)
// of sequence seq's context, entries of a sequence consecutive;
// first_part[i] is sequence i's first entry (first_part[num_seqs] = total).
// Every workgroup rescans the per-sequence entry counts in LDS, so one
// launch builds the whole plan.  Entries past the total get rows = 0.
__global__ __launch_bounds__(kPlanThreads) void attn_plan_kernel(
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

// Shared state of one workgroup: the entry's cache rows, each wave's
// partials.
template <int HQ>
struct AttnShared {
  int32_t rows[kEntryRows];
  float acc[kAttnWaves][HQ][kHeadDim];
  float m[kAttnWaves][HQ];
  float l[kAttnWaves][HQ];
};

// Partials of plan entry blockIdx.x, for every query head qh:
//   part_acc[entry][qh][d/2] = fp16 pair of sum_rows p * v[d] * 2^-k,
//   part_ml[entry][qh] = (m + k, l * 2^-k),
// with p = 2^(score - m) against the reference max m (log2 units), l the
// sum of the p, and k a per-head power of two that puts the largest
// magnitude in [2^14, 2^15) (a 12-bit mantissa for every value well above
// 2^-27 of the largest, no fp16 overflow).  Folding k into both m and l
// keeps the merge exact: both sums carry the same factor 2^(m + k - M).
// An entry without valid rows gives (-inf, 0) and zeros.
//
// Epilogue: each wave publishes its partials in LDS; after one barrier the
// waves split the query heads and merge and store them in parallel, which
// ends the workgroup (and frees its LDS for the next) sooner than one wave
// merging every head.
template <int HKV, int G, bool kHalf>
__global__ __launch_bounds__(kAttnThreads) NKV_ATTN_OCCUPANCY void attn_decode_partial_kernel(
    const uint16_t* __restrict__ q, int64_t q_seq_stride,
    const uint8_t* __restrict__ key_cache, const uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ tables, int64_t table_stride, int32_t block_size,
    int32_t num_blocks, const int4* __restrict__ plan, int32_t num_seqs, float scale_log2,
    uint32_t* __restrict__ part_acc, f32x2* __restrict__ part_ml) {
  constexpr int HQ = HKV * G;
  constexpr int NC = HKV >= 4 ? HKV / 4 : 1;   // kv heads per lane per row
  constexpr int TPI = HKV >= 4 ? 1 : 4 / HKV;  // rows per wavefront load
  constexpr int kRowBytes = HKV * kHeadBytes;
  static_assert(HQ <= kMaxQHeads && NC * G <= 4, "unsupported head layout");
  __shared__ AttnShared<HQ> sh;

  const int64_t part = blockIdx.x;
  const int4 entry = plan[part];
  const int32_t row0 = entry.x;
  const int32_t seq = entry.z;
  // Uniform exits; an empty cache (num_blocks == 0) has no row to read.
  if (entry.y <= 0 || seq < 0 || seq >= num_seqs || row0 < 0) return;
  const int32_t nrows = num_blocks > 0 ? min(entry.y, kEntryRows) : 0;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int slot = lane >> 4;
  const int sub = lane & 15;
  const int head0 = HKV >= 4 ? slot : slot % HKV;
  const int row_off = HKV >= 4 ? 0 : slot / HKV;

  // q first, so its loads overlap the block-id loads of the rows below.
  u32x4 qf[NC][G];
  const uint16_t* qs = q + static_cast<int64_t>(seq) * q_seq_stride;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int qh = (head0 + 4 * c) * G + g;
      qf[c][g] = *reinterpret_cast<const u32x4*>(qs + qh * kHeadDim + sub * 8);
    }
  }

  // Cache row of every context row of the entry; the block ids pass through
  // the merge buffer, which is idle until the loop below ends.
  static_assert(sizeof(sh.acc) >= kEntryRows * sizeof(int32_t), "block-id scratch too small");
  resolve_rows<kAttnThreads>(tables, table_stride, seq, row0, nrows, block_size, num_blocks,
                             reinterpret_cast<int32_t*>(&sh.acc[0][0][0]), sh.rows);

  float m[NC][G], l[NC][G], acc[NC][G][8];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      m[c][g] = -INFINITY;
      l[c][g] = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[c][g][j] = 0.f;
    }
  }

  // Each iteration a wave takes kAttnUnroll * TPI consecutive rows, and the
  // waves' groups are adjacent, so the workgroup sweeps its rows as one
  // front.
  constexpr int32_t kGroupRows = kAttnUnroll * TPI;
  for (int32_t r = wave * kGroupRows; r < nrows; r += kAttnWaves * kGroupRows) {
    u32x4 kw[kAttnUnroll][NC], vw[kAttnUnroll][NC];
    bool ok[kAttnUnroll];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const int32_t t = r + u * TPI + row_off;
      const int32_t cache_row = t < nrows ? sh.rows[t] : -1;
      ok[u] = cache_row >= 0;
      // A skipped row re-reads cache row 0 (in bounds: the cache is not
      // empty here), gets a -inf score and zeroed V words.
      const int64_t safe_row = ok[u] ? cache_row : 0;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int64_t off = safe_row * kRowBytes + (HKV >= 4 ? c * 1024 + lane * 16
                                                            : (lane & (16 * HKV - 1)) * 16);
#if NKV_ATTN_NT_LOADS
        kw[u][c] = load_stream(reinterpret_cast<const u32x4*>(key_cache + off));
        vw[u][c] = load_stream(reinterpret_cast<const u32x4*>(value_cache + off));
#else
        kw[u][c] = *reinterpret_cast<const u32x4*>(key_cache + off);
        vw[u][c] = *reinterpret_cast<const u32x4*>(value_cache + off);
#endif
      }
    }
    // A skipped row's bytes may be any bits (row 0 need not hold a written
    // row): its score is -inf below, and its V words are zeroed here, since
    // a zero weight times NaN or Inf would still reach the sums.
    bool group_ok = true;
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) group_ok = group_ok && ok[u];
    if (!__all(group_ok)) {
#pragma unroll
      for (int u = 0; u < kAttnUnroll; ++u) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (!ok[u]) vw[u][c] = u32x4{0u, 0u, 0u, 0u};
        }
      }
    }
    float s[kAttnUnroll][NC][G];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float d = row16_sum(dot8<kHalf>(kw[u][c], qf[c][g], 0.f));
          s[u][c][g] = ok[u] ? d * scale_log2 : -INFINITY;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float v[kAttnUnroll][8];
#pragma unroll
      for (int u = 0; u < kAttnUnroll; ++u) {
        v[u][0] = elem_lo<kHalf>(vw[u][c].x);
        v[u][1] = elem_hi<kHalf>(vw[u][c].x);
        v[u][2] = elem_lo<kHalf>(vw[u][c].y);
        v[u][3] = elem_hi<kHalf>(vw[u][c].y);
        v[u][4] = elem_lo<kHalf>(vw[u][c].z);
        v[u][5] = elem_hi<kHalf>(vw[u][c].z);
        v[u][6] = elem_lo<kHalf>(vw[u][c].w);
        v[u][7] = elem_hi<kHalf>(vw[u][c].w);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mt = s[0][c][g];
#pragma unroll
        for (int u = 1; u < kAttnUnroll; ++u) mt = fmaxf(mt, s[u][c][g]);
        // Also taken for the first valid rows (m = -inf, corr = 0).
        if (mt > m[c][g] + kRescaleLog2) {
          const float corr = exp2_fast(m[c][g] - mt);
          l[c][g] *= corr;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[c][g][j] *= corr;
          m[c][g] = mt;
        }
        if (m[c][g] == -INFINITY) continue;  // nothing valid yet for this row
        const float m_ref = m[c][g];
#pragma unroll
        for (int u = 0; u < kAttnUnroll; ++u) {
          const float p = exp2_fast(s[u][c][g] - m_ref);
          l[c][g] += p;
#pragma unroll
          for (int j = 0; j < 8; ++j) acc[c][g][j] = fmaf(p, v[u][j], acc[c][g][j]);
        }
      }
    }
  }

  // Rows of one wavefront load that share a kv head sit 16*HKV lanes apart
  // (HKV < 4): merge them so lanes with row_off == 0 hold the wave's result.
  if constexpr (TPI > 1) {
#pragma unroll
    for (int x = 16 * HKV; x < kWave; x <<= 1) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float mo = __shfl_xor(m[c][g], x, kWave);
          const float lo = __shfl_xor(l[c][g], x, kWave);
          const float mm = fmaxf(m[c][g], mo);
          const float fa = mm == -INFINITY ? 0.f : exp2_fast(m[c][g] - mm);
          const float fb = mm == -INFINITY ? 0.f : exp2_fast(mo - mm);
          l[c][g] = l[c][g] * fa + lo * fb;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float ao = __shfl_xor(acc[c][g][j], x, kWave);
            acc[c][g][j] = acc[c][g][j] * fa + ao * fb;
          }
          m[c][g] = mm;
        }
      }
    }
  }

  if (row_off == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int qh = (head0 + 4 * c) * G + g;
#pragma unroll
        for (int j = 0; j < 8; ++j) sh.acc[wave][qh][sub * 8 + j] = acc[c][g][j];
        if (sub == 0) {
          sh.m[wave][qh] = m[c][g];
          sh.l[wave][qh] = l[c][g];
        }
      }
    }
  }
  // Every wave's partials are in LDS after the barrier; each wave then
  // merges every kAttnWaves-th query head, two dims per lane, against the
  // largest reference, scales and stores it.
  __syncthreads();
  for (int qh = wave; qh < HQ; qh += kAttnWaves) {
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) mm = fmaxf(mm, sh.m[w][qh]);
    float a0 = 0.f, a1 = 0.f, lsum = 0.f;
    if (mm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        const float f = exp2_fast(sh.m[w][qh] - mm);
        a0 = fmaf(sh.acc[w][qh][2 * lane], f, a0);
        a1 = fmaf(sh.acc[w][qh][2 * lane + 1], f, a1);
        lsum = fmaf(sh.l[w][qh], f, lsum);
      }
    }
    emit_partial(part_acc + (part * HQ + qh) * (kHeadDim / 2), part_ml + part * HQ + qh, a0, a1,
                 mm, lsum, lane);
  }
}

// Grouped-query decode on MFMA.  With G = Hq / Hkv query heads per kv head
// the VALU kernel above spends 2 G FLOPs per cache byte on v_dot2 and fma
// (plus a DPP row sum per head), which outruns the memory time from G = 4
// on.  Here the G query heads of one kv head form the 16 columns of one
// MFMA tile (up to 16 heads, padding columns zero), so the arithmetic of a
// 16-key chunk is a fixed 13 MFMAs whatever G is:
//   * S^T = K Q^T: 4 x 16x16x32 (keys x heads, over 128 dims); a lane holds
//     head c16 and keys 4 g4 + i, which is exactly the B layout of a
//     16x16x16 MFMA over those keys, so P^T needs no shuffle;
//   * O^T += V^T P^T: 8 x 16x16x16 (dims x heads, over 16 keys), V^T from
//     the transposing LDS read; a ninth product against a row of ones sums
//     the same (rounded) weights;
//   * the online softmax is a 4-lane max per head and one exp2 per score.
// A workgroup owns one (plan entry, kv head).  Its wavefronts take the
// entry's 16-key chunks round-robin and run independently: each has a
// private ring of kDecSlots chunk buffers in LDS, filled by global_load_lds
// kDecSlots - 1 chunks ahead of the one it computes and waited for with a
// counted s_waitcnt (8 copies per chunk), so no barrier sits in the loop.
// The waves then merge through LDS and split the stores of the query heads,
// as above, in the same format, for the same reduce kernel.
// Invalid rows (block id missing or outside the cache, keys past the entry)
// copy cache row 0 into their slots; their scores are masked and their V
// rows zeroed before the product.
#ifndef NKV_DEC_WAVES
#define NKV_DEC_WAVES 4  // wavefronts per workgroup
#endif
#ifndef NKV_DEC_SLOTS
#define NKV_DEC_SLOTS 2  // 16-key chunk buffers per wavefront
#endif
#ifndef NKV_DEC_NT_LOADS
#define NKV_DEC_NT_LOADS 1  // stream K/V past the caches (nt)
#endif
constexpr int kDecWaves = NKV_DEC_WAVES;
constexpr int kDecThreads = kDecWaves * kWave;
constexpr int kDecSlots = NKV_DEC_SLOTS;
constexpr int kDecKeys = 16;                  // keys per chunk
constexpr int kDecChunkWords = kDecKeys * 16;  // 16-byte words per K or V chunk
constexpr int kDecCopies = 2 * kDecKeys / 4;   // copy instructions per chunk (K and V)
constexpr int kDecMaxGroup = 16;               // query heads per kv head (MFMA columns)
// Smallest G run on MFMA by default (smaller G: the VALU kernel).  With the
// kv head rotated over the XCDs the MFMA kernel is the faster one on every
// layout measured, G = 1 and 2 included (256-sequence decode step, one
// layer, whole calls: 16 q / 8 kv 547.8 against 560.6-561.1 us, 8 / 8
// 554.0-554.5 against 577.3-578.0, 8 / 4 289.9-290.0 against 302.5-303.6,
// 4 / 2 152.5-152.6 against 156.6-157.1), so it serves every layout.  The
// VALU kernel stays for the G <= 2 layouts it covers when NKV_DECODE_VALU=1
// is set in the environment (read on every call).
#ifndef NKV_DEC_MFMA_MIN_GROUP
#define NKV_DEC_MFMA_MIN_GROUP 1
#endif
constexpr int kDecMfmaMinGroup = NKV_DEC_MFMA_MIN_GROUP;
// G below which the VALU kernel runs when NKV_DECODE_VALU=1 asks for it.
constexpr int kDecValuMaxGroup = 2;
static_assert(kDecWaves == 2 || kDecWaves == 4 || kDecWaves == 8,
              "NKV_DEC_WAVES must be 2, 4 or 8");
static_assert(kDecSlots >= 2 && kDecSlots <= 4, "NKV_DEC_SLOTS must be in [2, 4]");

// One wavefront's LDS: its ring while it runs, its partials afterwards.
union DecWaveMem {
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
struct DecShared {
  DecWaveMem wave[kDecWaves];
  int32_t rows[(kEntryRows + kDecKeys - 1) / kDecKeys * kDecKeys];  // whole chunks
};

// s_waitcnt vmcnt(n) with the other counters left alone, and a compiler
// barrier for memory (the LDS reads after it must stay after it).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt is 6 bits");
  asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

template <bool kWide, bool kHalf>
__global__ __launch_bounds__(kDecThreads) void attn_decode_mfma_kernel(
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
  __shared__ DecShared sh;

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
  DecWaveMem& mine = sh.wave[wave];
  // LDS byte addresses of this wave's ring (uniform; the copies' M0 base).
  const uint32_t ring_k = lds_address(&sh.wave[0].ring.k[0][0]) +
                          static_cast<uint32_t>(wave) * sizeof(DecWaveMem);
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

// Merges the partials of (sequence, query head) pairs, one wavefront per
// pair and no LDS or barrier: lane i loads part i's (m + k, l 2^-k), and
// every lane loads its two dims (one fp16 pair) of up to kReduceBatch parts
// in the same round trip, so the merge waits for memory twice (the
// sequence's part range, then the parts) instead of three times.  The wave
// takes the parts' max with lane shuffles, weights and sums the parts in
// fp32 (part i's m and l come from lane i by shuffle) and divides once.  A
// context of more than kReduceBatch parts goes in batches, the running sums
// rescaled when a later batch raises the max.
constexpr int kReduceWaves = 4;  // pairs per workgroup
constexpr int kReduceThreads = kReduceWaves * kWave;
constexpr int kReduceBatch = 8;  // parts in flight per lane (contexts up to 6144 rows at 768 per part)

template <bool kHalf>
__global__ __launch_bounds__(kReduceThreads) void attn_decode_reduce_kernel(
    const uint32_t* __restrict__ part_acc, const f32x2* __restrict__ part_ml,
    const int32_t* __restrict__ first_part, int64_t capacity, int32_t num_seqs,
    int32_t num_q_heads, uint16_t* __restrict__ out, int64_t out_seq_stride) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t pair = static_cast<int64_t>(blockIdx.x) * kReduceWaves + wave;
  if (pair >= static_cast<int64_t>(num_seqs) * num_q_heads) return;  // whole waves; no barrier
  const int32_t seq = static_cast<int32_t>(pair / num_q_heads);
  const int32_t qh = static_cast<int32_t>(pair % num_q_heads);
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
  *reinterpret_cast<uint32_t*>(out + static_cast<int64_t>(seq) * out_seq_stride +
                               qh * kHeadDim + 2 * lane) = packed;
}

using PartialKernel = void (*)(const uint16_t*, int64_t, const uint8_t*, const uint8_t*,
                               const int32_t*, int64_t, int32_t, int32_t, const int4*, int32_t,
                               float, uint32_t*, f32x2*);

template <bool kHalf>
PartialKernel partial_kernel_for(int64_t hkv, int64_t g) {
#define NKV_ATTN_CASE(H, GG) \
  if (hkv == H && g == GG) return attn_decode_partial_kernel<H, GG, kHalf>;
  // One or two query heads per kv head; more go to the MFMA kernel.
  NKV_ATTN_CASE(8, 1)
  NKV_ATTN_CASE(8, 2)
  NKV_ATTN_CASE(4, 1)
  NKV_ATTN_CASE(4, 2)
  NKV_ATTN_CASE(2, 1)
  NKV_ATTN_CASE(2, 2)
  NKV_ATTN_CASE(1, 1)
  NKV_ATTN_CASE(1, 2)
#undef NKV_ATTN_CASE
  return nullptr;
}

using DecodeMfmaKernel = void (*)(const uint16_t*, int64_t, const uint8_t*, const uint8_t*,
                                   const int32_t*, int64_t, int32_t, int32_t, int32_t, int32_t,
                                   const int4*, int32_t, float, uint32_t*, f32x2*);

DecodeMfmaKernel mfma_kernel_for(bool wide, bool half) {
  if (wide) return half ? attn_decode_mfma_kernel<true, true> : attn_decode_mfma_kernel<true, false>;
  return half ? attn_decode_mfma_kernel<false, true> : attn_decode_mfma_kernel<false, false>;
}

}  // namespace
}  // namespace nkv

extern "C" int64_t nkv_attention_entry_rows(int64_t block_size) {
  return block_size > 0 ? nkv::attention_entry_rows(block_size) : 0;
}

extern "C" int64_t nkv_attention_plan_capacity(int64_t total_tokens, int64_t num_seqs,
                                               int64_t block_size) {
  if (total_tokens < 0 || num_seqs < 0 || block_size <= 0) return 0;
  const int64_t rows = nkv::attention_entry_rows(block_size);
  return (total_tokens + rows - 1) / rows + num_seqs;
}

extern "C" int64_t nkv_attention_workspace_bytes(int64_t capacity, int64_t num_q_heads,
                                                 int64_t head_dim) {
  if (capacity < 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  // per (entry, query head): head_dim fp16 sums and a float2 (m + k, l * 2^-k)
  return capacity * num_q_heads * (head_dim * 2 + 8);
}

extern "C" int nkv_build_attention_plan(const int32_t* cu_seqlens_k, int64_t num_seqs,
                                        int64_t block_size, void* plan, int64_t capacity,
                                        int32_t* first_part, void* stream) {
  using namespace nkv;
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: num_seqs=%lld outside [0, %d]",
                    static_cast<long long>(num_seqs), NKV_MAX_PLAN_SEQS);
  }
  if (block_size <= 0 || block_size > INT32_MAX || capacity < 0 || capacity > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: bad block_size or capacity");
  }
  if (!first_part || (num_seqs > 0 && !cu_seqlens_k) || (capacity > 0 && !plan)) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: plan must be 16-byte aligned");
  }
  const int64_t blocks = capacity > 0 ? (capacity + kPlanThreads - 1) / kPlanThreads : 1;
  const size_t lds = (static_cast<size_t>(num_seqs) + 1 + kPlanThreads / kWave + 1) *
                     sizeof(int32_t);
  attn_plan_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kPlanThreads), lds,
                     static_cast<hipStream_t>(stream)>>>(
      cu_seqlens_k, static_cast<int32_t>(num_seqs),
      static_cast<int32_t>(attention_entry_rows(block_size)), static_cast<int4*>(plan),
      capacity, first_part);
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
  // MFMA from kDecMfmaMinGroup query heads per kv head on (every layout by
  // default), and for every layout the VALU kernels do not cover; the VALU
  // kernel below that, or for G <= 2 when NKV_DECODE_VALU=1.
  const char* valu_env = std::getenv("NKV_DECODE_VALU");
  const bool valu_requested = valu_env != nullptr && valu_env[0] == '1' && valu_env[1] == '\0';
  const int64_t mfma_min_group = valu_requested ? kDecValuMaxGroup + 1 : kDecMfmaMinGroup;
  bool use_mfma = group >= mfma_min_group && group <= kDecMaxGroup;
  PartialKernel kernel = nullptr;
  if (!use_mfma) {
    kernel = half ? partial_kernel_for<true>(num_kv_heads, group)
                  : partial_kernel_for<false>(num_kv_heads, group);
    if (kernel == nullptr && group <= kDecMaxGroup) use_mfma = true;
  }
  if (!use_mfma && kernel == nullptr) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: unsupported head layout %lld kv x %lld q "
                    "(at most %d query heads per kv head)",
                    static_cast<long long>(num_kv_heads), static_cast<long long>(num_q_heads),
                    kDecMaxGroup);
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS || capacity < 0 || capacity > INT32_MAX ||
      block_size <= 0 || num_blocks < 0 || num_blocks * block_size > INT32_MAX ||
      table_stride < 0 || q_seq_stride < num_q_heads * head_dim ||
      out_seq_stride < num_q_heads * head_dim) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: bad sizes or strides");
  }
  // Both kernels rely on scale > 0: the MFMA kernel takes the chunk max of
  // the raw scores (masked rows at -inf) before scaling, which commutes with
  // a positive scale only (0 or a negative scale would turn masked rows into
  // NaN or +inf weights).
  if (!std::isfinite(scale) || !(scale > 0.f)) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: scale must be finite and positive");
  }
  if (num_seqs == 0) return NKV_OK;
  const int64_t need = nkv_attention_workspace_bytes(capacity, num_q_heads, head_dim);
  if (workspace_bytes < need) {
    return nkv_fail(NKV_E_CAPACITY,
                    "nkv_paged_attention_decode: workspace of %lld bytes < %lld needed",
                    static_cast<long long>(workspace_bytes), static_cast<long long>(need));
  }
  if (!q || !key_cache || !value_cache || !first_part || !out ||
      (capacity > 0 && (!plan || !workspace || (table_stride > 0 && !block_tables)))) {
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
  if (use_mfma && (capacity * num_kv_heads > INT32_MAX || num_kv_heads * head_dim * 2 > INT32_MAX)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: plan too long for the grid");
  }
  auto* part_acc = static_cast<uint32_t*>(workspace);  // fp16 pairs
  auto* part_ml = reinterpret_cast<f32x2*>(part_acc + capacity * num_q_heads * head_dim / 2);
  if (capacity > 0 && use_mfma) {
    // byte offsets into a cache past 4 GiB need 64-bit addresses
    const bool wide = num_blocks * block_size * num_kv_heads * head_dim * 2 > UINT32_MAX;
    mfma_kernel_for(wide, half)<<<dim3(static_cast<unsigned>(capacity * num_kv_heads)),
                                  dim3(kDecThreads), 0, s>>>(
        static_cast<const uint16_t*>(q), q_seq_stride, static_cast<const uint8_t*>(key_cache),
        static_cast<const uint8_t*>(value_cache), block_tables, table_stride,
        static_cast<int32_t>(block_size), static_cast<int32_t>(num_blocks),
        static_cast<int32_t>(num_kv_heads), static_cast<int32_t>(group),
        static_cast<const int4*>(plan), static_cast<int32_t>(num_seqs), scale_log2, part_acc,
        part_ml);
    if (int rc = nkv_check_launch("nkv_paged_attention_decode (MFMA partials)")) return rc;
  } else if (capacity > 0) {
    kernel<<<dim3(static_cast<unsigned>(capacity)), dim3(kAttnThreads), 0, s>>>(
        static_cast<const uint16_t*>(q), q_seq_stride, static_cast<const uint8_t*>(key_cache),
        static_cast<const uint8_t*>(value_cache), block_tables, table_stride,
        static_cast<int32_t>(block_size), static_cast<int32_t>(num_blocks),
        static_cast<const int4*>(plan), static_cast<int32_t>(num_seqs), scale_log2, part_acc,
        part_ml);
    if (int rc = nkv_check_launch("nkv_paged_attention_decode (partials)")) return rc;
  }
  // one wavefront per (sequence, query head) pair, kReduceWaves pairs per workgroup
  const int64_t pairs = num_seqs * num_q_heads;
  const dim3 reduce_grid(static_cast<unsigned>((pairs + kReduceWaves - 1) / kReduceWaves));
  if (half) {
    attn_decode_reduce_kernel<true><<<reduce_grid, dim3(kReduceThreads), 0, s>>>(
        part_acc, part_ml, first_part, capacity, static_cast<int32_t>(num_seqs),
        static_cast<int32_t>(num_q_heads), static_cast<uint16_t*>(out), out_seq_stride);
  } else {
    attn_decode_reduce_kernel<false><<<reduce_grid, dim3(kReduceThreads), 0, s>>>(
        part_acc, part_ml, first_part, capacity, static_cast<int32_t>(num_seqs),
        static_cast<int32_t>(num_q_heads), static_cast<uint16_t*>(out), out_seq_stride);
  }
  return nkv_check_launch("nkv_paged_attention_decode (reduce)");
}
