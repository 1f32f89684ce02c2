// Paged-attention decode: one query token per sequence attends over its
// context straight from the paged KV cache, so the context is read once and
// never gathered.  This is the consumer the reference's decode path calls
// (flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens, block_table,
// softmax_scale, causal=True), nanovllm/layers/attention.py:122-130); its
// numerical reference is SDPAAttention's decode branch
// (attention.py:284-300: gather, then scaled_dot_product_attention with
// enable_gqa, query head j reading kv head j / (Hq / Hkv)).
//
// Split-K ("flash decoding"): one workgroup per (sequence, cache block)
// computes, for every query head, the block's softmax partials
// (running max m, sum l, unnormalised output acc), and a reduce kernel
// merges the partials of each (sequence, query head).
//
// Mapping inside a workgroup (256 threads, head_dim 128, bf16):
//   * a 16-lane DPP row owns one (row, kv head): each lane holds 8 dims
//     (16 bytes), so a wavefront instruction reads 1 KiB of consecutive
//     cache bytes (coalesced, non-temporal);
//   * q.k for the G = Hq/Hkv query heads of that kv head is 4 v_dot2 on
//     packed bf16 pairs plus a 4-step DPP row sum (fp32);
//   * an online softmax in fp32 with exp2 (scale * log2 e folded in),
//     updated once per 4 rows per wave;
//   * the 4 waves split the block's rows and merge their partials in LDS.
// Decode attention moves ~2 bytes per FLOP pair and has only G = 2..8 query
// rows per kv head, so it is bound by HBM reads; an MFMA tile (16 rows)
// would idle 75-94% of its lanes, while the VALU work here is well under the
// memory time and overlaps it across waves.
#include <cmath>

#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / kWave;
constexpr int kHeadDim = 128;
constexpr int kHeadBytes = kHeadDim * 2;  // bf16
constexpr int kAttnUnroll = 4;
constexpr int kMaxQHeads = 16;

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// One v_dot2 on a packed bf16 pair.  The words arrive as scalars on purpose:
// __builtin_bit_cast applied directly to an ext_vector component (a.y) is
// lowered by this clang to component 0 for every component.
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, a),
                                         __builtin_bit_cast(bf16x2v, b), acc, false);
}

__device__ __forceinline__ float dot8_bf16(u32x4 a, u32x4 b, float acc) {
  acc = dot2_bf16(a.x, b.x, acc);
  acc = dot2_bf16(a.y, b.y, acc);
  acc = dot2_bf16(a.z, b.z, acc);
  acc = dot2_bf16(a.w, b.w, acc);
  return acc;
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

// fp32 -> bf16, round to nearest even (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu) != 0u) return 0x7FC0;
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Plan entry (from launch_block_plan with chunk_rows = block_size):
// x = first cache row of the block (-1 if the block id is invalid), y = the
// rows' offset in the sequence's context (unused), z = rows, w = sequence.
template <int HKV, int G>
__global__ __launch_bounds__(kAttnThreads) void attn_decode_partial_kernel(
    const uint16_t* __restrict__ q, int64_t q_seq_stride,
    const uint8_t* __restrict__ key_cache, const uint8_t* __restrict__ value_cache,
    const int4* __restrict__ plan, int32_t num_seqs, int64_t cache_rows,
    int32_t block_size, float scale_log2, float* __restrict__ part_acc,
    float2* __restrict__ part_ml) {
  constexpr int HQ = HKV * G;
  constexpr int NC = HKV >= 4 ? HKV / 4 : 1;   // kv heads per lane per row
  constexpr int TPI = HKV >= 4 ? 1 : 4 / HKV;  // rows per wavefront load
  constexpr int kRowBytes = HKV * kHeadBytes;
  static_assert(HQ <= kMaxQHeads && NC * G <= 8, "unsupported head layout");

  const int4 entry = plan[blockIdx.x];
  const int32_t nrows = entry.z;
  const int32_t seq = entry.w;
  if (nrows <= 0 || seq < 0 || seq >= num_seqs) return;
  const int64_t src_row = entry.x;
  const bool block_ok = src_row >= 0 && src_row + nrows <= cache_rows;
  const int32_t valid_rows = block_ok ? nrows : 0;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int slot = lane >> 4;
  const int sub = lane & 15;
  const int head0 = HKV >= 4 ? slot : slot % HKV;
  const int row_off = HKV >= 4 ? 0 : slot / HKV;

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

  // Rows [r_begin, r_end) of the block belong to this wave (multiples of TPI).
  const int32_t per_wave =
      (block_size + kAttnWaves * TPI - 1) / (kAttnWaves * TPI) * TPI;
  const int32_t r_begin = wave * per_wave;
  const int32_t r_end = min(valid_rows, r_begin + per_wave);
  const uint8_t* kb = key_cache + (block_ok ? src_row : 0) * kRowBytes;
  const uint8_t* vb = value_cache + (block_ok ? src_row : 0) * kRowBytes;

  for (int32_t r = r_begin; r < r_end; r += TPI * kAttnUnroll) {
    u32x4 kw[kAttnUnroll][NC], vw[kAttnUnroll][NC];
    bool ok[kAttnUnroll];
#pragma unroll
    for (int u = 0; u < kAttnUnroll; ++u) {
      const int32_t row_base = r + u * TPI;
      ok[u] = row_base + row_off < r_end;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        kw[u][c] = u32x4{0u, 0u, 0u, 0u};
        vw[u][c] = u32x4{0u, 0u, 0u, 0u};
        if (ok[u]) {
          const int64_t off = static_cast<int64_t>(row_base) * kRowBytes + c * 1024 + lane * 16;
          kw[u][c] = load_stream(reinterpret_cast<const u32x4*>(kb + off));
          vw[u][c] = load_stream(reinterpret_cast<const u32x4*>(vb + off));
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
          const float d = row16_sum(dot8_bf16(kw[u][c], qf[c][g], 0.f));
          s[u][c][g] = ok[u] ? d * scale_log2 : -INFINITY;
        }
      }
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      float v[kAttnUnroll][8];
#pragma unroll
      for (int u = 0; u < kAttnUnroll; ++u) {
        v[u][0] = bf16_lo(vw[u][c].x);
        v[u][1] = bf16_hi(vw[u][c].x);
        v[u][2] = bf16_lo(vw[u][c].y);
        v[u][3] = bf16_hi(vw[u][c].y);
        v[u][4] = bf16_lo(vw[u][c].z);
        v[u][5] = bf16_hi(vw[u][c].z);
        v[u][6] = bf16_lo(vw[u][c].w);
        v[u][7] = bf16_hi(vw[u][c].w);
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float mt = s[0][c][g];
#pragma unroll
        for (int u = 1; u < kAttnUnroll; ++u) mt = fmaxf(mt, s[u][c][g]);
        const float m_new = fmaxf(m[c][g], mt);
        if (m_new == -INFINITY) continue;  // nothing valid yet for this row
        const float corr = exp2_fast(m[c][g] - m_new);
        l[c][g] *= corr;
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[c][g][j] *= corr;
        m[c][g] = m_new;
#pragma unroll
        for (int u = 0; u < kAttnUnroll; ++u) {
          const float p = exp2_fast(s[u][c][g] - m_new);
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

  __shared__ float s_acc[kAttnWaves][HQ][kHeadDim];
  __shared__ float s_m[kAttnWaves][HQ];
  __shared__ float s_l[kAttnWaves][HQ];
  if (row_off == 0) {
#pragma unroll
    for (int c = 0; c < NC; ++c) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const int qh = (head0 + 4 * c) * G + g;
#pragma unroll
        for (int j = 0; j < 8; ++j) s_acc[wave][qh][sub * 8 + j] = acc[c][g][j];
        if (sub == 0) {
          s_m[wave][qh] = m[c][g];
          s_l[wave][qh] = l[c][g];
        }
      }
    }
  }
  __syncthreads();
  const int64_t part = blockIdx.x;
  for (int idx = threadIdx.x; idx < HQ * kHeadDim; idx += kAttnThreads) {
    const int qh = idx / kHeadDim;
    const int d = idx - qh * kHeadDim;
    float mm = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) mm = fmaxf(mm, s_m[w][qh]);
    float a = 0.f, lsum = 0.f;
    if (mm != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        const float f = exp2_fast(s_m[w][qh] - mm);
        a = fmaf(s_acc[w][qh][d], f, a);
        lsum = fmaf(s_l[w][qh], f, lsum);
      }
    }
    part_acc[(part * HQ + qh) * kHeadDim + d] = a;
    if (d == 0) part_ml[part * HQ + qh] = make_float2(mm, lsum);
  }
}

// Merges the partials of one (sequence, query head): thread = one dim.
__global__ __launch_bounds__(kHeadDim) void attn_decode_reduce_kernel(
    const float* __restrict__ part_acc, const float2* __restrict__ part_ml,
    const int32_t* __restrict__ first_part, int64_t capacity, int32_t num_q_heads,
    uint16_t* __restrict__ out, int64_t out_seq_stride) {
  const int32_t seq = blockIdx.x;
  const int32_t qh = blockIdx.y;
  const int32_t d = threadIdx.x;
  const int64_t p0 = max(0, first_part[seq]);
  const int64_t p1 = min(capacity, static_cast<int64_t>(first_part[seq + 1]));
  float mm = -INFINITY;
  for (int64_t p = p0; p < p1; ++p) mm = fmaxf(mm, part_ml[p * num_q_heads + qh].x);
  float a = 0.f, lsum = 0.f;
  if (mm != -INFINITY) {
    for (int64_t p = p0; p < p1; ++p) {
      const float2 ml = part_ml[p * num_q_heads + qh];
      const float f = exp2_fast(ml.x - mm);
      a = fmaf(part_acc[(p * num_q_heads + qh) * kHeadDim + d], f, a);
      lsum = fmaf(ml.y, f, lsum);
    }
  }
  const float o = lsum > 0.f ? a / lsum : 0.f;
  out[static_cast<int64_t>(seq) * out_seq_stride + qh * kHeadDim + d] = to_bf16(o);
}

using PartialKernel = void (*)(const uint16_t*, int64_t, const uint8_t*, const uint8_t*,
                               const int4*, int32_t, int64_t, int32_t, float, float*, float2*);

PartialKernel partial_kernel_for(int64_t hkv, int64_t g) {
#define NKV_ATTN_CASE(H, GG) \
  if (hkv == H && g == GG) return attn_decode_partial_kernel<H, GG>;
  NKV_ATTN_CASE(8, 1)
  NKV_ATTN_CASE(8, 2)
  NKV_ATTN_CASE(4, 1)
  NKV_ATTN_CASE(4, 2)
  NKV_ATTN_CASE(4, 4)
  NKV_ATTN_CASE(2, 1)
  NKV_ATTN_CASE(2, 2)
  NKV_ATTN_CASE(2, 4)
  NKV_ATTN_CASE(2, 8)
  NKV_ATTN_CASE(1, 1)
  NKV_ATTN_CASE(1, 2)
  NKV_ATTN_CASE(1, 4)
  NKV_ATTN_CASE(1, 8)
#undef NKV_ATTN_CASE
  return nullptr;
}

}  // namespace
}  // namespace nkv

extern "C" int64_t nkv_attention_plan_capacity(int64_t total_tokens, int64_t num_seqs,
                                               int64_t block_size) {
  if (total_tokens < 0 || num_seqs < 0 || block_size <= 0) return 0;
  return (total_tokens + block_size - 1) / block_size + num_seqs;
}

extern "C" int64_t nkv_attention_workspace_bytes(int64_t capacity, int64_t num_q_heads,
                                                 int64_t head_dim) {
  if (capacity < 0 || num_q_heads <= 0 || head_dim <= 0) return 0;
  return capacity * num_q_heads * (head_dim * 4 + 8);
}

extern "C" int nkv_build_attention_plan(const int32_t* block_tables, int64_t table_stride,
                                        const int32_t* cu_seqlens_k, int64_t num_seqs,
                                        int64_t block_size, int64_t num_blocks, void* plan,
                                        int64_t capacity, int32_t* first_part,
                                        void* stream) {
  using namespace nkv;
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: num_seqs=%lld outside [0, %d]",
                    static_cast<long long>(num_seqs), NKV_MAX_PLAN_SEQS);
  }
  if (block_size <= 0 || num_blocks < 0 || num_blocks * block_size > INT32_MAX ||
      capacity < 0 || capacity > INT32_MAX || table_stride < 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: bad geometry or capacity");
  }
  if (!first_part || (num_seqs > 0 && (!block_tables || !cu_seqlens_k)) ||
      (capacity > 0 && !plan)) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_attention_plan: plan must be 16-byte aligned");
  }
  return launch_block_plan(block_tables, table_stride, cu_seqlens_k, num_seqs, INT32_MAX,
                           block_size, block_size, num_blocks, static_cast<int32_t*>(plan),
                           capacity, first_part, static_cast<hipStream_t>(stream),
                           "nkv_build_attention_plan");
}

extern "C" int nkv_paged_attention_decode(
    const void* q, int64_t q_seq_stride, const void* key_cache, const void* value_cache,
    const void* plan, int64_t capacity, const int32_t* first_part, int64_t num_seqs,
    int64_t num_kv_heads, int64_t num_q_heads, int64_t head_dim, int64_t block_size,
    int64_t num_blocks, float scale, int32_t dtype, void* workspace, int64_t workspace_bytes,
    void* out, int64_t out_seq_stride, void* stream) {
  using namespace nkv;
  if (dtype != NKV_DTYPE_BFLOAT16) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: only bfloat16 is supported");
  }
  if (head_dim != kHeadDim) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: head_dim must be %d", kHeadDim);
  }
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: num_q_heads must be a multiple of num_kv_heads");
  }
  const PartialKernel kernel = partial_kernel_for(num_kv_heads, num_q_heads / num_kv_heads);
  if (kernel == nullptr) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: unsupported head layout %lld kv x %lld q "
                    "(kv heads 1/2/4/8, at most %d query heads)",
                    static_cast<long long>(num_kv_heads), static_cast<long long>(num_q_heads),
                    kMaxQHeads);
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS || capacity < 0 || capacity > INT32_MAX ||
      block_size <= 0 || num_blocks < 0 || num_blocks * block_size > INT32_MAX ||
      q_seq_stride < num_q_heads * head_dim || out_seq_stride < num_q_heads * head_dim) {
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
  if (!q || !key_cache || !value_cache || !first_part || !out || (capacity > 0 && (!plan || !workspace))) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_decode: null pointer");
  }
  if ((reinterpret_cast<uint64_t>(q) | reinterpret_cast<uint64_t>(key_cache) |
       reinterpret_cast<uint64_t>(value_cache) | reinterpret_cast<uint64_t>(plan) |
       reinterpret_cast<uint64_t>(workspace) | static_cast<uint64_t>(q_seq_stride * 2)) % 16 != 0 ||
      reinterpret_cast<uint64_t>(out) % 2 != 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_decode: q/caches/plan/workspace must be 16-byte aligned");
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* part_acc = static_cast<float*>(workspace);
  auto* part_ml = reinterpret_cast<float2*>(part_acc + capacity * num_q_heads * head_dim);
  const float scale_log2 = scale * 1.4426950408889634f;  // log2(e)
  if (capacity > 0) {
    kernel<<<dim3(static_cast<unsigned>(capacity)), dim3(kAttnThreads), 0, s>>>(
        static_cast<const uint16_t*>(q), q_seq_stride, static_cast<const uint8_t*>(key_cache),
        static_cast<const uint8_t*>(value_cache), static_cast<const int4*>(plan),
        static_cast<int32_t>(num_seqs), num_blocks * block_size,
        static_cast<int32_t>(block_size), scale_log2, part_acc, part_ml);
    if (int rc = nkv_check_launch("nkv_paged_attention_decode (partials)")) return rc;
  }
  attn_decode_reduce_kernel<<<dim3(static_cast<unsigned>(num_seqs),
                                   static_cast<unsigned>(num_q_heads)),
                              dim3(kHeadDim), 0, s>>>(
      part_acc, part_ml, first_part, capacity, static_cast<int32_t>(num_q_heads),
      static_cast<uint16_t*>(out), out_seq_stride);
  return nkv_check_launch("nkv_paged_attention_decode (reduce)");
}
