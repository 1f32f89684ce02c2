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
// whole blocks), one workgroup per entry computes softmax partials for every
// query head (reference max m, weight sum l, unnormalised output), and a
// reduce kernel merges the partials of each (sequence, query head).
//
// Mapping inside a workgroup (8 waves, head_dim 128, bf16 or fp16):
//   * the entry's cache rows are resolved once through the block table into
//     LDS (invalid block ids give rows that are skipped);
//   * a 16-lane DPP row owns one (row, kv head): each lane holds 8 dims
//     (16 bytes), so a wavefront instruction reads 1 KiB of consecutive
//     cache bytes (coalesced, non-temporal); the waves take interleaved
//     groups of rows, so the workgroup sweeps its rows as one front;
//   * q.k for the G = Hq/Hkv query heads of that kv head is 4 v_dot2 on
//     packed bf16 / fp16 pairs plus a 4-step DPP row sum (fp32);
//   * an online softmax in fp32 with exp2 (scale * log2 e folded in);
//   * the waves merge in LDS without a barrier: the last one to arrive
//     stores the entry's partials (fp16 sums with a power-of-two scale).
// Decode attention moves ~2 bytes per FLOP pair and has only G = 1..8 query
// rows per kv head, so it is bound by HBM reads; an MFMA tile (16 rows)
// would idle most of its lanes, while the VALU work here stays under the
// memory time and overlaps it across waves.
#include <cmath>

#include "nkv_common.h"

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
constexpr int kMaxQHeads = 32;  // the waves' LDS merge buffer: 4 KiB per query head
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

// Shared state of one workgroup: the entry's cache rows, each wave's
// partials, and the count of waves that have published theirs.
template <int HQ>
struct AttnShared {
  int32_t rows[kEntryRows];
  float acc[kAttnWaves][HQ][kHeadDim];
  float m[kAttnWaves][HQ];
  float l[kAttnWaves][HQ];
  uint32_t arrived;
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
// Epilogue without a barrier: each wave publishes its partials in LDS and
// bumps an arrival counter; the last wave to arrive merges and stores them,
// the others exit at once, so their slots go to the next workgroup instead
// of idling until the slowest wave's loads return.
// kRowHeads: kv heads in a cache row (HKV unless the layout is run in parts
// of HKV heads).
template <int HKV, int G, bool kHalf, int kRowHeads = HKV>
__global__ __launch_bounds__(kAttnThreads) NKV_ATTN_OCCUPANCY void attn_decode_partial_kernel(
    const uint16_t* __restrict__ q, int64_t q_seq_stride,
    const uint8_t* __restrict__ key_cache, const uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ tables, int64_t table_stride, int32_t block_size,
    int32_t num_blocks, const int4* __restrict__ plan, int32_t num_seqs, float scale_log2,
    uint32_t* __restrict__ part_acc, f32x2* __restrict__ part_ml) {
  constexpr int HQ = HKV * G;
  constexpr int NC = HKV >= 4 ? HKV / 4 : 1;   // kv heads per lane per row
  constexpr int TPI = HKV >= 4 ? 1 : 4 / HKV;  // rows per wavefront load
  constexpr int kRowBytes = kRowHeads * kHeadBytes;
  static_assert(HQ <= kMaxQHeads && NC * G <= 8, "unsupported head layout");
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

  // Cache row of every context row of the entry, -1 where the block id is
  // missing from the table or outside the cache.
  for (int32_t t = threadIdx.x; t < nrows; t += kAttnThreads) {
    const int32_t ctx = row0 + t;
    const int32_t logical = ctx / block_size;
    int32_t cache_row = -1;
    if (logical < table_stride) {
      const int32_t block = tables[static_cast<int64_t>(seq) * table_stride + logical];
      if (block >= 0 && block < num_blocks) cache_row = block * block_size + ctx % block_size;
    }
    sh.rows[t] = cache_row;
  }
  if (threadIdx.x == 0) sh.arrived = 0u;
  __syncthreads();  // rows resolved, counter zero, before any wave reads or arrives

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
      // empty here) and gets a -inf score, i.e. zero weight.
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
  // Publish (release), count the arrival; the wave that arrives last sees
  // every other wave's partials after the acquire.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  uint32_t before = 0u;
  if (lane == 0) {
    before = __hip_atomic_fetch_add(&sh.arrived, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  before = __builtin_amdgcn_readfirstlane(before);
  if (before != kAttnWaves - 1) return;  // whole wavefront; no barrier follows
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

  // Per query head, two dims per lane: merge the waves against the largest
  // reference, scale, store.
  for (int qh = 0; qh < HQ; ++qh) {
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
    float amax = fmaxf(fabsf(a0), fabsf(a1));
#pragma unroll
    for (int x = kWave / 2; x > 0; x >>= 1) amax = fmaxf(amax, __shfl_xor(amax, x, kWave));
    const int e = static_cast<int>((__float_as_uint(amax) >> 23) & 0xFFu) - 127;
    const int k = amax > 0.f ? min(112, max(-112, e - 14)) : 0;
    const float down = __uint_as_float(static_cast<uint32_t>(127 - k) << 23);
    const uint32_t packed =
        static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a0 * down))) |
        (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<_Float16>(a1 * down)))
         << 16);
    store_stream(part_acc + (part * HQ + qh) * (kHeadDim / 2) + lane, packed);
    if (lane == 0) {
      store_stream(part_ml + part * HQ + qh, f32x2{mm + static_cast<float>(k), lsum * down});
    }
  }
}

// Merges the partials of one (sequence, query head): the 4 waves of the
// workgroup take the max of the parts' references together, then each walks
// a quarter of the parts (two dims per lane from one fp16 pair, unrolled so
// several loads are in flight), and wave 0 adds the four sums and divides
// once.
constexpr int kReduceWaves = 4;
constexpr int kReduceThreads = kReduceWaves * kWave;

template <bool kHalf>
__global__ __launch_bounds__(kReduceThreads) void attn_decode_reduce_kernel(
    const uint32_t* __restrict__ part_acc, const f32x2* __restrict__ part_ml,
    const int32_t* __restrict__ first_part, int64_t capacity, int32_t num_q_heads,
    uint16_t* __restrict__ out, int64_t out_seq_stride) {
  __shared__ float s_max[kReduceWaves];
  __shared__ float s_acc[kReduceWaves][kHeadDim];
  __shared__ float s_l[kReduceWaves];
  const int32_t seq = blockIdx.x;
  const int32_t qh = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t p0 = max(0, first_part[seq]);
  const int64_t p1 = min(capacity, static_cast<int64_t>(first_part[seq + 1]));

  float mm = -INFINITY;
  for (int64_t p = p0 + threadIdx.x; p < p1; p += kReduceThreads) {
    mm = fmaxf(mm, part_ml[p * num_q_heads + qh].x);
  }
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) mm = fmaxf(mm, __shfl_xor(mm, d, kWave));
  if (lane == 0) s_max[wave] = mm;
  __syncthreads();
#pragma unroll
  for (int w = 0; w < kReduceWaves; ++w) mm = fmaxf(mm, s_max[w]);

  float ax = 0.f, ay = 0.f, lsum = 0.f;
  if (mm != -INFINITY) {
#pragma unroll 8
    for (int64_t p = p0 + wave; p < p1; p += kReduceWaves) {
      const f32x2 ml = part_ml[p * num_q_heads + qh];  // (m + k, l * 2^-k)
      const uint32_t v = part_acc[(p * num_q_heads + qh) * (kHeadDim / 2) + lane];
      const float f = exp2_fast(ml.x - mm);
      ax = fmaf(half_lo(v), f, ax);
      ay = fmaf(half_hi(v), f, ay);
      lsum = fmaf(ml.y, f, lsum);
    }
  }
  s_acc[wave][2 * lane] = ax;
  s_acc[wave][2 * lane + 1] = ay;
  if (lane == 0) s_l[wave] = lsum;
  __syncthreads();
  if (wave != 0) return;  // no barrier follows
  ax = ay = lsum = 0.f;
#pragma unroll
  for (int w = 0; w < kReduceWaves; ++w) {
    ax += s_acc[w][2 * lane];
    ay += s_acc[w][2 * lane + 1];
    lsum += s_l[w];
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
  // Every layout with G <= 8 query heads per kv head (G <= 4 with 8 kv
  // heads: a lane keeps 2 kv heads x G query heads in registers).
  NKV_ATTN_CASE(8, 1)
  NKV_ATTN_CASE(8, 2)
  NKV_ATTN_CASE(8, 3)
  NKV_ATTN_CASE(8, 4)
  NKV_ATTN_CASE(4, 1)
  NKV_ATTN_CASE(4, 2)
  NKV_ATTN_CASE(4, 3)
  NKV_ATTN_CASE(4, 4)
  NKV_ATTN_CASE(4, 5)
  NKV_ATTN_CASE(4, 6)
  NKV_ATTN_CASE(4, 7)
  NKV_ATTN_CASE(4, 8)
  NKV_ATTN_CASE(2, 1)
  NKV_ATTN_CASE(2, 2)
  NKV_ATTN_CASE(2, 3)
  NKV_ATTN_CASE(2, 4)
  NKV_ATTN_CASE(2, 5)
  NKV_ATTN_CASE(2, 6)
  NKV_ATTN_CASE(2, 7)
  NKV_ATTN_CASE(2, 8)
  NKV_ATTN_CASE(1, 1)
  NKV_ATTN_CASE(1, 2)
  NKV_ATTN_CASE(1, 3)
  NKV_ATTN_CASE(1, 4)
  NKV_ATTN_CASE(1, 5)
  NKV_ATTN_CASE(1, 6)
  NKV_ATTN_CASE(1, 7)
  NKV_ATTN_CASE(1, 8)
#undef NKV_ATTN_CASE
  return nullptr;
}
// 8 kv heads with 5 to 8 query heads each (40 to 64 query heads): run as
// two parts of 4 kv heads, each reading its half of every cache row.
template <bool kHalf>
PartialKernel split_partial_kernel_for(int64_t g) {
  switch (g) {
    case 5: return attn_decode_partial_kernel<4, 5, kHalf, 8>;
    case 6: return attn_decode_partial_kernel<4, 6, kHalf, 8>;
    case 7: return attn_decode_partial_kernel<4, 7, kHalf, 8>;
    case 8: return attn_decode_partial_kernel<4, 8, kHalf, 8>;
    default: return nullptr;
  }
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
  PartialKernel kernel = half ? partial_kernel_for<true>(num_kv_heads, group)
                              : partial_kernel_for<false>(num_kv_heads, group);
  int64_t parts = 1;  // launches, each over num_kv_heads / parts kv heads
  if (kernel == nullptr && num_kv_heads == 8) {
    kernel = half ? split_partial_kernel_for<true>(group) : split_partial_kernel_for<false>(group);
    parts = 2;
  }
  if (kernel == nullptr) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: unsupported head layout %lld kv x %lld q "
                    "(kv heads 1/2/4/8, at most 8 query heads per kv head)",
                    static_cast<long long>(num_kv_heads), static_cast<long long>(num_q_heads));
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS || capacity < 0 || capacity > INT32_MAX ||
      block_size <= 0 || num_blocks < 0 || num_blocks * block_size > INT32_MAX ||
      table_stride < 0 || q_seq_stride < num_q_heads * head_dim ||
      out_seq_stride < num_q_heads * head_dim) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: bad sizes or strides");
  }
  if (!std::isfinite(scale)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: scale must be finite");
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
  // Each part covers num_kv_heads / parts kv heads and their query heads:
  // q, out and the caches advance by that many heads; the parts run one
  // after the other on the stream and share the workspace.
  const int64_t part_q_heads = num_q_heads / parts;
  auto* part_acc = static_cast<uint32_t*>(workspace);  // fp16 pairs
  auto* part_ml = reinterpret_cast<f32x2*>(part_acc + capacity * part_q_heads * head_dim / 2);
  for (int64_t p = 0; p < parts; ++p) {
    const int64_t q_off = p * part_q_heads * head_dim;                        // elements
    const int64_t kv_off = p * (num_kv_heads / parts) * head_dim * 2;         // bytes
    if (capacity > 0) {
      kernel<<<dim3(static_cast<unsigned>(capacity)), dim3(kAttnThreads), 0, s>>>(
          static_cast<const uint16_t*>(q) + q_off, q_seq_stride,
          static_cast<const uint8_t*>(key_cache) + kv_off,
          static_cast<const uint8_t*>(value_cache) + kv_off, block_tables, table_stride,
          static_cast<int32_t>(block_size), static_cast<int32_t>(num_blocks),
          static_cast<const int4*>(plan), static_cast<int32_t>(num_seqs), scale_log2, part_acc,
          part_ml);
      if (int rc = nkv_check_launch("nkv_paged_attention_decode (partials)")) return rc;
    }
    const dim3 reduce_grid(static_cast<unsigned>(num_seqs), static_cast<unsigned>(part_q_heads));
    uint16_t* part_out = static_cast<uint16_t*>(out) + q_off;
    if (half) {
      attn_decode_reduce_kernel<true><<<reduce_grid, dim3(kReduceThreads), 0, s>>>(
          part_acc, part_ml, first_part, capacity, static_cast<int32_t>(part_q_heads), part_out,
          out_seq_stride);
    } else {
      attn_decode_reduce_kernel<false><<<reduce_grid, dim3(kReduceThreads), 0, s>>>(
          part_acc, part_ml, first_part, capacity, static_cast<int32_t>(part_q_heads), part_out,
          out_seq_stride);
    }
    if (int rc = nkv_check_launch("nkv_paged_attention_decode (reduce)")) return rc;
  }
  return NKV_OK;
}
