// Paged-attention prefill: causal attention of a chunk of query tokens per
// sequence over that sequence's context, read straight from the paged KV
// cache through its block table.  This is the prefill call of the
// reference's Flash path (flash_attn_varlen_func(q, k_cache, v_cache,
// cu_seqlens_q, cu_seqlens_k, ..., causal=True, block_table=...),
// nanovllm/layers/attention.py:95-116); its numerical reference is the SDPA
// prefill (attention.py:226-282: gather each request's keys, then SDPA with
// the prefix-causal mask of :155-161).  Query j of a request with Lq queries
// and Lk context rows sits at position Lk - Lq + j and sees keys
// [0, Lk - Lq + j]; query head h reads kv head h / (Hq / Hkv).
//
// The work is GEMM-shaped (each K/V tile serves 128 query rows), so both
// products run on MFMA (v_mfma_f32_16x16x32_bf16 / _f16, fp32 accumulation):
//   * a workgroup owns 128 query rows of one (sequence, kv head): the
//     (token, query head) pairs of 128 / G consecutive tokens and the
//     G = Hq / Hkv query heads that share the kv head, token-major;
//     each of its 4 waves owns 32 of those rows (two 16-row blocks);
//   * the keys stream in tiles of 64, K and V copied straight from the cache
//     into LDS (global_load_lds, swizzled 16-byte chunks), one tile in
//     flight while the previous one is computed; the V^T operands come from
//     the transposing LDS read of gfx950;
//   * scores are computed transposed, S^T = K Q^T, so that a lane's
//     accumulators all belong to ONE query row: the online softmax needs
//     only a 4-lane max per row, the P^T operand of O^T = V^T P^T comes
//     straight from the score registers (the transposing reads deliver V^T
//     in the same key order), and the output rescale is a per-lane factor;
//   * P is rounded to the input type (bf16 or fp16) for the second product,
//     as flash attention does, and the row sum is taken from the same
//     rounded weights;
//   * the query tiles of one kv head run on one XCD (shared L2).
// Invalid block ids (outside [0, num_blocks), or past the table) drop their
// keys, as in the decode kernel.
#include <cmath>
#include <type_traits>

#include "nkv_common.h"
#include "nkv_mfma.h"

namespace nkv {
namespace {

#ifndef NKV_PF_WAVES
#define NKV_PF_WAVES 4  // wavefronts per workgroup (4 or 8), 32 query rows each
#endif
constexpr int kPfWaves = NKV_PF_WAVES;
static_assert(kPfWaves == 4 || kPfWaves == 8, "NKV_PF_WAVES must be 4 or 8");
// Two wavefronts per SIMD: two 4-wave workgroups per CU, or one of 8.
constexpr int kPfBlocksPerCU = 8 / kPfWaves;
constexpr int kPfThreads = kPfWaves * kWave;
constexpr int kPfRows = kPfWaves * 32;  // query rows per workgroup
constexpr int kPfKeys = 64;             // keys per tile
constexpr int kPfDim = 128;             // head_dim
constexpr int kPfPlanThreads = 1024;

// Lazy softmax reference (log2 units): weights stay <= 2^8 before the final
// division, far from fp32 / bf16 / fp16 overflow.
constexpr float kRescaleLog2 = 8.f;

// K and V tiles, double-buffered, copied straight from global memory into
// LDS by global_load_lds (one wavefront instruction fills 1 KiB of
// consecutive LDS: 4 keys x 256 B; the source address of each lane picks
// the chunk that belongs at its position), in the swizzled layout of
// k_index / v_index.  Each buffer is its own __shared__ array, and the loop
// body is compiled once per buffer parity, so the compiler can tell the tile
// being read from the one being copied into.
constexpr int kTileChunks = kPfKeys * 16;  // 16-byte chunks per K or V tile

// Plan: one int4 {seq, token0, tokens, 0} per workgroup: tokens [token0,
// token0 + tokens) of sequence seq's queries, tokens <= tile_tokens.
// Entries past the total get tokens = 0.  The tiles are listed longest
// first (most visible keys: the keys of a tile's last query), so that the
// longest workgroups start first and the short ones fill the tail; ties in
// plan order.  Plans of up to kPfSortMax tiles are sorted in LDS by one
// workgroup (bitonic); longer ones list each sequence's tiles last tile
// first, sequence after sequence.
#ifndef NKV_PF_SETPRIO
#define NKV_PF_SETPRIO 1  // raise the wave's priority over its MFMA block (0: never)
#endif
#ifndef NKV_PF_SORT_MAX
#define NKV_PF_SORT_MAX 2048  // longest plan sorted in LDS (0: never sort)
#endif
constexpr int kPfSortMax = NKV_PF_SORT_MAX;

__global__ __launch_bounds__(kPfPlanThreads) void prefill_plan_kernel(
    const int32_t* __restrict__ cu_seqlens_q, const int32_t* __restrict__ cu_seqlens_k,
    int32_t num_seqs, int32_t tile_tokens, int4* __restrict__ plan, int64_t capacity,
    int32_t sort) {
  extern __shared__ int32_t s_mem[];
  int32_t* s_first = s_mem;               // [num_seqs + 1]
  int32_t* s_tmp = s_mem + num_seqs + 1;  // [kPfPlanThreads / 64 + 1]
  lds_exclusive_scan<kPfPlanThreads>(
      num_seqs,
      [&](int32_t i) {
        const int32_t len = cu_seqlens_q[i + 1] - cu_seqlens_q[i];
        return len > 0 ? (len + tile_tokens - 1) / tile_tokens : 0;
      },
      s_first, s_tmp);
  const int64_t total = s_first[num_seqs];
  // Entry e in sequence order: sequence i's tiles, last tile first.
  auto entry_of = [&](int32_t e) {
    const int32_t i = owner_of(s_first, num_seqs, e);
    const int32_t tiles = s_first[i + 1] - s_first[i];
    const int32_t t0 = (tiles - 1 - (e - s_first[i])) * tile_tokens;
    const int32_t len = cu_seqlens_q[i + 1] - cu_seqlens_q[i];
    return make_int4(i, t0, min(tile_tokens, len - t0), 0);
  };
  if (sort && total <= kPfSortMax) {  // one workgroup (the launch makes sure)
    // Sort keys: (2^31 - 1 - visible keys) << 32 | e, ascending; padding last.
    const int32_t key_offset = (num_seqs + kPfPlanThreads / 64 + 3) & ~1;  // 8-byte aligned
    uint64_t* s_key = reinterpret_cast<uint64_t*>(s_mem + key_offset);
    int32_t n2 = 1;
    while (n2 < total) n2 <<= 1;
    for (int32_t e = threadIdx.x; e < n2; e += kPfPlanThreads) {
      uint64_t key = ~uint64_t{0};
      if (e < total) {
        const int4 en = entry_of(e);
        const int32_t lq = cu_seqlens_q[en.x + 1] - cu_seqlens_q[en.x];
        const int32_t lk = cu_seqlens_k[en.x + 1] - cu_seqlens_k[en.x];
        const int32_t visible = max(0, lk - lq + en.y + en.z);
        key = (static_cast<uint64_t>(0x7FFFFFFF - visible) << 32) | static_cast<uint32_t>(e);
      }
      s_key[e] = key;
    }
    for (int32_t k = 2; k <= n2; k <<= 1) {
      for (int32_t j = k >> 1; j > 0; j >>= 1) {
        __syncthreads();
        for (int32_t i = threadIdx.x; i < n2; i += kPfPlanThreads) {
          const int32_t partner = i ^ j;
          if (partner > i) {
            const uint64_t a = s_key[i], b = s_key[partner];
            if ((a > b) == ((i & k) == 0)) {
              s_key[i] = b;
              s_key[partner] = a;
            }
          }
        }
      }
    }
    __syncthreads();
    for (int64_t e = threadIdx.x; e < capacity; e += kPfPlanThreads) {
      plan[e] = e < total ? entry_of(static_cast<int32_t>(s_key[e] & 0xFFFFFFFFu))
                          : make_int4(0, 0, 0, 0);
    }
    return;
  }
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kPfPlanThreads;
  for (int64_t e = static_cast<int64_t>(blockIdx.x) * kPfPlanThreads + threadIdx.x; e < capacity;
       e += stride) {
    plan[e] = e < total ? entry_of(static_cast<int32_t>(e)) : make_int4(0, 0, 0, 0);
  }
}

// Where one sequence's context rows live: its block table and the cache
// geometry.  Power-of-two block sizes map rows with shifts.
struct ContextMap {
  const int32_t* table;
  int64_t table_stride;
  int32_t block_size;
  int32_t block_shift;  // log2(block_size), or -1 when it is not a power of two
  int32_t num_blocks;
  int32_t num_keys;     // rows past this are never read

  // Physical cache row of context row t, or -1 when t is past num_keys or
  // the table, or its block id is outside [0, num_blocks).  Split in two so
  // that the table load can be issued early and consumed late.
  __device__ __forceinline__ int32_t block_of(int32_t t) const {
    const int32_t logical = block_shift >= 0 ? t >> block_shift : t / block_size;
    if (t >= num_keys || logical >= table_stride) return -1;
    return table[logical];
  }
  __device__ __forceinline__ int32_t row_in(int32_t t, int32_t block) const {
    if (block < 0 || block >= num_blocks) return -1;
    const int32_t offset = block_shift >= 0 ? t & (block_size - 1) : t % block_size;
    return block * block_size + offset;  // num_blocks * block_size <= INT32_MAX
  }
  __device__ __forceinline__ int32_t row(int32_t t) const { return row_in(t, block_of(t)); }
};

// Wavefront 0 resolves the 64 rows of the tile starting at key0 (one per
// lane, from the block id its lane loaded) and whether any is invalid.
__device__ __forceinline__ void resolve_rows(int32_t* rows, int32_t* invalid, const ContextMap& map,
                                             int32_t key0, int32_t block, int lane) {
  const int32_t row = map.row_in(key0 + lane, block);
  rows[lane] = row;
  const bool any_invalid = __any(row < 0);
  if (lane == 0) *invalid = any_invalid ? 1 : 0;
}

// This wavefront's share of the copies of one K or V tile: 64 / waves
// consecutive keys, 4 keys per instruction; lane l copies 16-byte chunk
// swizzle(l % 16) of key l / 16.  The block rows are read first, so the
// copies issue back to back.  Lanes of invalid rows copy nothing (the K
// scores of such keys are masked and their V zeroed).  kWide: byte offsets
// into the cache may exceed 32 bits, so lanes form 64-bit addresses.
template <bool kWide, bool kValue>
__device__ __forceinline__ void issue_copies(const u32x4* dst, const int32_t* rows,
                                             const uint8_t* head_base, uint32_t row_bytes,
                                             int wave, int lane) {
  constexpr int kKeysPerWave = kPfKeys / kPfWaves;
  constexpr int kCopies = kKeysPerWave / 4;
  const int pos = lane & 15;
  int32_t row[kCopies];
#pragma unroll
  for (int i = 0; i < kCopies; ++i) row[i] = rows[kKeysPerWave * wave + 4 * i + (lane >> 4)];
#pragma unroll
  for (int i = 0; i < kCopies; ++i) {
    const int key0 = kKeysPerWave * wave + 4 * i;
    const int key = key0 + (lane >> 4);
    const uint32_t chunk = 16u * (kValue ? pos ^ ((key & 7) << 1) : pos ^ (key & 15));
    const uint32_t lds_dst = lds_address(dst) + key0 * 256;  // wave is uniform
    if (row[i] >= 0) {
      if (kWide) {
        lds_copy16(head_base + static_cast<int64_t>(row[i]) * row_bytes + chunk, lds_dst);
      } else {
        lds_copy16(head_base, static_cast<uint32_t>(row[i]) * row_bytes + chunk, lds_dst);
      }
    }
  }
}

// Workgroups are handed to the 8 XCDs round-robin by linear id (id % 8), and
// each XCD has its own L2.  The grid is one-dimensional and its ids are
// mapped so that the query tiles of one kv head run on one XCD, or on 8 / H
// of them when there are H < 8 kv heads: the tiles that read the same K/V
// rows then share an L2 instead of each XCD fetching them again.  Within an
// XCD the tiles keep the plan's order (each sequence's last tile first).
//   layout 1 (H a multiple of 8): XCD x runs kv heads x, x + 8, ... in turn;
//   layout 2 (H divides 8): XCD x runs kv head x / R, R = 8 / H, and every
//     R-th plan entry from x % R; the grid is 8 ceil(capacity / R), and ids
//     past the plan exit;
//   layout 0 (any other H): kv head fastest, no XCD grouping.
constexpr int kXcds = 8;
struct TileId {
  int32_t entry;    // plan entry
  int32_t kv_head;
};

__device__ __forceinline__ TileId tile_of(uint32_t id, int32_t num_kv_heads, int32_t capacity,
                                          int32_t layout) {
  const int32_t x = static_cast<int32_t>(id % kXcds);
  const int32_t turn = static_cast<int32_t>(id / kXcds);  // dispatch order within the XCD
  if (layout == 1) return TileId{turn % capacity, x + kXcds * (turn / capacity)};
  if (layout == 2) {
    const int32_t per_head = kXcds / num_kv_heads;
    return TileId{turn * per_head + x % per_head, x / per_head};
  }
  return TileId{static_cast<int32_t>(id / num_kv_heads), static_cast<int32_t>(id % num_kv_heads)};
}

template <int G, bool kWide, bool kHalf>
__global__ __launch_bounds__(kPfThreads, kPfBlocksPerCU) void attn_prefill_kernel(
    const uint16_t* __restrict__ q, int64_t q_token_stride,
    const uint8_t* __restrict__ key_cache, const uint8_t* __restrict__ value_cache,
    const int32_t* __restrict__ tables, int64_t table_stride, int32_t block_size,
    int32_t block_shift, int32_t num_blocks, int32_t num_kv_heads,
    const int32_t* __restrict__ cu_seqlens_q, const int32_t* __restrict__ cu_seqlens_k,
    const int4* __restrict__ plan, int32_t capacity, int32_t xcd_layout, int32_t num_seqs,
    float scale_log2, uint16_t* __restrict__ out, int64_t out_token_stride) {
  constexpr int kTileTokens = kPfRows / G;
  typedef Elem<kHalf> E;
  typedef typename E::T T;
  typedef typename E::X8 X8;
  typedef typename E::X4 X4;
  __shared__ u32x4 k_buf0[kTileChunks];
  __shared__ u32x4 k_buf1[kTileChunks];
  __shared__ u32x4 v_buf0[kTileChunks];
  __shared__ u32x4 v_buf1[kTileChunks];
  __shared__ int32_t rows_buf[4][kPfKeys];  // physical row of each key of a tile, -1 if invalid
  __shared__ int32_t invalid_buf[4];        // whether a tile has an invalid row

  const TileId id = tile_of(blockIdx.x, num_kv_heads, capacity, xcd_layout);
  if (id.entry >= capacity) return;
  const int4 entry = plan[id.entry];
  const int32_t seq = entry.x;
  const int32_t tok0 = entry.y;
  const int32_t ntok = entry.z;
  const int32_t kh = id.kv_head;
  // Uniform exits for empty or malformed entries.
  if (ntok <= 0 || ntok > kTileTokens || seq < 0 || seq >= num_seqs || tok0 < 0) return;
  const int32_t q_begin = cu_seqlens_q[seq];
  const int32_t lq = cu_seqlens_q[seq + 1] - q_begin;
  const int32_t lk = cu_seqlens_k[seq + 1] - cu_seqlens_k[seq];
  if (lk < lq || tok0 + ntok > lq) return;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // uniform: scalar registers
  const int lane = tid % kWave;
  const int c16 = lane & 15;  // the lane's query row inside a 16-row block
  const int g4 = lane >> 4;   // which quarter of the MFMA k dimension the lane holds
  const uint32_t row_bytes = static_cast<uint32_t>(num_kv_heads) * kPfDim * 2;
  const uint8_t* const k_head = key_cache + static_cast<int64_t>(kh) * kPfDim * 2;
  const uint8_t* const v_head = value_cache + static_cast<int64_t>(kh) * kPfDim * 2;
  // keys the last row sees (<= lk); every row sees at least first_row_keys
  const int32_t num_keys = lk - lq + tok0 + ntok;
  const int32_t first_row_keys = lk - lq + tok0 + 1;
  const ContextMap map{tables + static_cast<int64_t>(seq) * table_stride, table_stride,
                       block_size, block_shift, num_blocks, num_keys};

  // Q^T operands (B of S^T = K Q^T): lane holds row m, dims 32 * dc + 8 * g4 .. +8.
  X8 qb[2][4];
  int32_t limit[2];  // last visible key of the lane's row, -1 for rows past the tile
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const int m = wave * 32 + mb * 16 + c16;
    const int t = m / G;
    const bool row_ok = t < ntok;
    limit[mb] = row_ok ? lk - lq + tok0 + t : -1;
    const uint16_t* qrow = q + static_cast<int64_t>(q_begin + tok0 + (row_ok ? t : 0)) *
                                   q_token_stride + (kh * G + m % G) * kPfDim;
#pragma unroll
    for (int dc = 0; dc < 4; ++dc) {
      u32x4 v = {0u, 0u, 0u, 0u};
      if (row_ok) v = *reinterpret_cast<const u32x4*>(qrow + 32 * dc + 8 * g4);
      qb[mb][dc] = __builtin_bit_cast(X8, v);
    }
  }

  const int32_t num_tiles = (num_keys + kPfKeys - 1) / kPfKeys;
  float row_max[2] = {-INFINITY, -INFINITY};
  // O^T blocks: dims 16 * db + 4 * g4 + i of row m.  Block 8 multiplies P
  // by a row of ones (dim 128 of an extended V^T), so its first dim holds
  // the row's weight sum, taken from the same bf16 weights as the output.
  f32x4 acc[9][2];
#pragma unroll
  for (int db = 0; db < 9; ++db) {
    acc[db][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[db][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const T one = c16 == 0 ? static_cast<T>(1.f) : static_cast<T>(0.f);
  const X8 ones = {one, one, one, one, one, one, one, one};

  // Software pipeline: tile t computes the softmax and PV of tile t and
  // the scores of tile t + 1, so the score MFMAs can issue between the
  // softmax's VALU instructions.  K is copied two tiles ahead (K(t + 2)
  // into the buffer of K(t), read by the scores of tile t during tile
  // t - 1), V one tile ahead.  Rows are resolved three tiles ahead, from
  // block ids loaded one tile before that (slots rotate over 4).
  int32_t ahead_block = -1;  // wavefront 0: block id of its lane's key in the next tile to resolve
  if (wave == 0) {
    // The four block-id loads issue together, so the workgroup's start waits
    // for one round trip through the table, not one per tile.
    int32_t first_blocks[3];
#pragma unroll
    for (int i = 0; i < 3; ++i) first_blocks[i] = i < num_tiles ? map.block_of(i * kPfKeys + lane) : -1;
    if (num_tiles > 3) ahead_block = map.block_of(3 * kPfKeys + lane);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      if (i < num_tiles) {
        resolve_rows(rows_buf[i], &invalid_buf[i], map, i * kPfKeys, first_blocks[i], lane);
      }
    }
  }
  __syncthreads();
  issue_copies<kWide, false>(k_buf0, rows_buf[0], k_head, row_bytes, wave, lane);
  issue_copies<kWide, true>(v_buf0, rows_buf[0], v_head, row_bytes, wave, lane);
  if (num_tiles > 1) issue_copies<kWide, false>(k_buf1, rows_buf[1], k_head, row_bytes, wave, lane);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  const int tr_key = 4 * g4 + ((lane >> 2) & 3);  // key this lane addresses in a V^T read (of 16)
  const int tr_dim = 4 * (lane & 3);              // first dim it addresses, within 16

  // S^T = K Q^T over one tile: block (kb, mb) holds keys 16 kb + 4 g4 + i of row m.
  auto scores = [&](const u32x4* k_tile, f32x4 (&s)[4][2]) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      s[kb][0] = f32x4{0.f, 0.f, 0.f, 0.f};
      s[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int dc = 0; dc < 4; ++dc) {
        const X8 a = __builtin_bit_cast(X8, k_tile[k_index(16 * kb + c16, 4 * dc + g4)]);
        s[kb][0] = E::mfma(a, qb[0][dc], s[kb][0]);
        s[kb][1] = E::mfma(a, qb[1][dc], s[kb][1]);
      }
    }
  };
  f32x4 st[4][2];
  scores(k_buf0, st);

  auto tile_step = [&](auto parity, int32_t tile) {
    constexpr int kCur = decltype(parity)::value;  // tile % 2
    u32x4* const k_this = kCur == 0 ? k_buf0 : k_buf1;  // held K(tile); receives K(tile + 2)
    u32x4* const k_next = kCur == 0 ? k_buf1 : k_buf0;  // K(tile + 1)
    u32x4* const v_cur = kCur == 0 ? v_buf0 : v_buf1;
    u32x4* const v_next = kCur == 0 ? v_buf1 : v_buf0;
    const int32_t key0 = tile * kPfKeys;
    const int slot = tile & 3;
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's copies of K(tile + 1), V(tile) have landed
    __syncthreads();                // ... and everyone's; tile - 1 is consumed
    const bool has_invalid = invalid_buf[slot] != 0;
    if (has_invalid) {  // zero V of invalid rows (not copied: the buffer holds an older tile)
#pragma unroll
      for (int i = 0; i < kTileChunks / kPfThreads; ++i) {
        const int idx = i * kPfThreads + tid;
        if (rows_buf[slot][idx >> 4] < 0) v_cur[idx] = u32x4{0u, 0u, 0u, 0u};
      }
      __syncthreads();
    }
    // The block ids used here landed with the wait above; those loaded
    // now land with the next tile's.
    if (wave == 0 && tile + 3 < num_tiles) {
      const int s3 = (tile + 3) & 3;
      resolve_rows(rows_buf[s3], &invalid_buf[s3], map, key0 + 3 * kPfKeys, ahead_block, lane);
      if (tile + 4 < num_tiles) ahead_block = map.block_of(key0 + 4 * kPfKeys + lane);
    }
    if (tile + 2 < num_tiles) {
      issue_copies<kWide, false>(k_this, rows_buf[(tile + 2) & 3], k_head, row_bytes, wave, lane);
    }
    if (tile + 1 < num_tiles) {
      issue_copies<kWide, true>(v_next, rows_buf[(tile + 1) & 3], v_head, row_bytes, wave, lane);
    }
    // A tile is plain when every row sees all its keys and all are valid:
    // its scores need no mask.
    const bool plain = !has_invalid && key0 + kPfKeys <= first_row_keys;

    // Online softmax per row (exp2 units): mask, max and the rare rescale.
    const int4* rows_now = reinterpret_cast<const int4*>(rows_buf[slot]);
    float ref[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
      if (!plain) {  // hide keys past the row's limit or in invalid rows
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          const int4 r = rows_now[4 * kb + g4];  // rows of keys 16 kb + 4 g4 + i
          const int32_t row[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (key0 + 16 * kb + 4 * g4 + i > limit[mb] || row[i] < 0) st[kb][mb][i] = -INFINITY;
          }
        }
      }
      float local = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int i = 0; i < 4; ++i) local = fmaxf(local, st[kb][mb][i]);
      local = row4_max(local) * scale_log2;  // scale > 0, so the max commutes with it
      // The row's reference max moves only when a score passes it by more
      // than kRescaleLog2 (always for the first visible score), so the
      // rescale of the accumulators is rare after the first tiles.
      const bool move = local > row_max[mb] + kRescaleLog2;
      if (__any(move)) {
        const float m_new = move ? local : row_max[mb];
        const float alpha = move ? __builtin_amdgcn_exp2f(row_max[mb] - m_new) : 1.f;
#pragma unroll
        for (int db = 0; db < 9; ++db) acc[db][mb] *= alpha;  // 0 when the old reference was -inf
        row_max[mb] = m_new;
      }
      // A row with nothing visible yet keeps the reference -inf: its
      // weights are 0 (hidden scores are -inf too).
      ref[mb] = row_max[mb] == -INFINITY ? INFINITY : row_max[mb];
    }

    // Weights of this tile, then the scores of the next tile.  After the
    // last tile the scores read a stale buffer and are dropped.
    X8 pb[2][2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        X8 w;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          w[i] = static_cast<T>(
              __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * c][mb][i], scale_log2, -ref[mb])));
          w[4 + i] = static_cast<T>(
              __builtin_amdgcn_exp2f(__builtin_fmaf(st[2 * c + 1][mb][i], scale_log2, -ref[mb])));
        }
        pb[c][mb] = w;
      }
    }
#if NKV_PF_SETPRIO
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(1);  // this wave's MFMA phase goes first on the SIMD
    __builtin_amdgcn_sched_barrier(0);
#endif
    scores(k_next, st);
    // Scheduler order for the scores: four K operand reads ahead, then
    // each read's two MFMAs with the next read.
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (i < 12) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // the PV product is scheduled on its own

    // O^T += V^T P^T.  Step c covers keys 32 c .. +32 in the order the P^T
    // operand holds them: slots 0-3 = keys 32c + 4 g4 + j, slots 4-7 = keys
    // 32c + 16 + 4 g4 + j; the transposing reads deliver V^T in that order.
#pragma unroll
    for (int db = 0; db < 8; ++db) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const u32x2 lo = v_tr_read(v_cur, 32 * c + tr_key, 16 * db + tr_dim);
        const u32x2 hi = v_tr_read(v_cur, 32 * c + 16 + tr_key, 16 * db + tr_dim);
        const X8 a = __builtin_bit_cast(X8, u32x4{lo.x, lo.y, hi.x, hi.y});
        acc[db][0] = E::mfma(a, pb[c][0], acc[db][0]);
        acc[db][1] = E::mfma(a, pb[c][1], acc[db][1]);
      }
    }
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      acc[8][0] = E::mfma(ones, pb[c][0], acc[8][0]);
      acc[8][1] = E::mfma(ones, pb[c][1], acc[8][1]);
    }
#if NKV_PF_SETPRIO
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
    __builtin_amdgcn_sched_barrier(0);
#endif
  };
  for (int32_t tile = 0; tile < num_tiles; tile += 2) {
    tile_step(std::integral_constant<int, 0>{}, tile);
    if (tile + 1 < num_tiles) tile_step(std::integral_constant<int, 1>{}, tile + 1);
  }

  // Normalise and store: the row's weight sum sits in the g4 == 0 lane.
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
    const float total = row4_sum(g4 == 0 ? acc[8][mb][0] : 0.f);
    const int m = wave * 32 + mb * 16 + c16;
    const int t = m / G;
    if (t >= ntok) continue;
    const float inv = total > 0.f ? 1.f / total : 0.f;
    uint16_t* orow = out + static_cast<int64_t>(q_begin + tok0 + t) * out_token_stride +
                     (kh * G + m % G) * kPfDim;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const f32x4 v = acc[db][mb];
      const X4 w = {static_cast<T>(v.x * inv), static_cast<T>(v.y * inv),
                    static_cast<T>(v.z * inv), static_cast<T>(v.w * inv)};
      *reinterpret_cast<X4*>(orow + 16 * db + 4 * g4) = w;
    }
  }
}

using PrefillKernel = void (*)(const uint16_t*, int64_t, const uint8_t*, const uint8_t*,
                               const int32_t*, int64_t, int32_t, int32_t, int32_t, int32_t,
                               const int32_t*, const int32_t*, const int4*, int32_t, int32_t,
                               int32_t, float, uint16_t*, int64_t);

template <bool kWide, bool kHalf>
PrefillKernel prefill_kernel_for(int64_t group) {
  switch (group) {
    case 1: return attn_prefill_kernel<1, kWide, kHalf>;
    case 2: return attn_prefill_kernel<2, kWide, kHalf>;
    case 3: return attn_prefill_kernel<3, kWide, kHalf>;
    case 4: return attn_prefill_kernel<4, kWide, kHalf>;
    case 5: return attn_prefill_kernel<5, kWide, kHalf>;
    case 6: return attn_prefill_kernel<6, kWide, kHalf>;
    case 7: return attn_prefill_kernel<7, kWide, kHalf>;
    case 8: return attn_prefill_kernel<8, kWide, kHalf>;
    default: return nullptr;
  }
}

}  // namespace
}  // namespace nkv

extern "C" int64_t nkv_prefill_tile_tokens(int64_t group) {
  // 128 query rows per workgroup: 128 / G whole tokens (with G = 3, 5, 6
  // or 7 the last 128 % G rows idle).
  return group >= 1 && group <= 8 ? nkv::kPfRows / group : 0;
}

extern "C" int64_t nkv_prefill_plan_capacity(int64_t total_q_tokens, int64_t num_seqs,
                                             int64_t group) {
  const int64_t tile = nkv_prefill_tile_tokens(group);
  if (total_q_tokens < 0 || num_seqs < 0 || tile == 0) return 0;
  return (total_q_tokens + tile - 1) / tile + num_seqs;
}

extern "C" int nkv_build_prefill_plan(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                      int64_t num_seqs, int64_t group, void* plan,
                                      int64_t capacity, void* stream) {
  using namespace nkv;
  const int64_t tile = nkv_prefill_tile_tokens(group);
  if (tile == 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_prefill_plan: query heads per kv head must be "
                                   "1 to 8 (got %lld)", static_cast<long long>(group));
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS || capacity < 0 || capacity > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_prefill_plan: num_seqs=%lld or capacity=%lld "
                                   "out of range", static_cast<long long>(num_seqs),
                    static_cast<long long>(capacity));
  }
  if (capacity == 0) return NKV_OK;
  if (!plan || (num_seqs > 0 && (!cu_seqlens_q || !cu_seqlens_k))) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_prefill_plan: null pointer");
  }
  if (reinterpret_cast<uint64_t>(plan) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_build_prefill_plan: plan must be 16-byte aligned");
  }
  // Plans that fit the LDS sort are built by one workgroup, longest tile
  // first; longer ones by a grid, in sequence order.
  const bool sort = capacity <= kPfSortMax;
  const int64_t blocks = sort ? 1 : (capacity + kPfPlanThreads - 1) / kPfPlanThreads;
  const size_t scan_ints = static_cast<size_t>(num_seqs) + 1 + kPfPlanThreads / kWave + 1;
  const size_t lds = sort ? ((scan_ints + 1) & ~size_t{1}) * sizeof(int32_t) +
                                kPfSortMax * sizeof(uint64_t)
                          : scan_ints * sizeof(int32_t);
  prefill_plan_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(kPfPlanThreads), lds,
                        static_cast<hipStream_t>(stream)>>>(
      cu_seqlens_q, cu_seqlens_k, static_cast<int32_t>(num_seqs), static_cast<int32_t>(tile),
      static_cast<int4*>(plan), capacity, sort ? 1 : 0);
  return nkv_check_launch("nkv_build_prefill_plan");
}

extern "C" int nkv_paged_attention_prefill(
    const void* q, int64_t q_token_stride, const void* key_cache, const void* value_cache,
    const int32_t* block_tables, int64_t table_stride, const int32_t* cu_seqlens_q,
    const int32_t* cu_seqlens_k, const void* plan, int64_t capacity, int64_t num_seqs,
    int64_t num_kv_heads, int64_t num_q_heads, int64_t head_dim, int64_t block_size,
    int64_t num_blocks, float scale, int32_t dtype, void* out, int64_t out_token_stride,
    void* stream) {
  using namespace nkv;
  if (dtype != NKV_DTYPE_BFLOAT16 && dtype != NKV_DTYPE_FLOAT16) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_prefill: only bfloat16 and float16 are supported");
  }
  const bool half = dtype == NKV_DTYPE_FLOAT16;
  if (head_dim != kPfDim) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_prefill: head_dim must be %d", kPfDim);
  }
  if (num_kv_heads <= 0 || num_q_heads <= 0 || num_q_heads % num_kv_heads != 0 ||
      num_kv_heads > 65535) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_prefill: num_q_heads must be a multiple of num_kv_heads");
  }
  if (nkv_prefill_tile_tokens(num_q_heads / num_kv_heads) == 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_prefill: %lld query heads per kv head (1 to 8 "
                    "supported)", static_cast<long long>(num_q_heads / num_kv_heads));
  }
  if (num_seqs < 0 || num_seqs > NKV_MAX_PLAN_SEQS || capacity < 0 || capacity > INT32_MAX ||
      block_size <= 0 || num_blocks < 0 || num_blocks * block_size > INT32_MAX ||
      table_stride < 0 || q_token_stride < num_q_heads * head_dim ||
      out_token_stride < num_q_heads * head_dim) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_prefill: bad sizes or strides");
  }
  if (!std::isfinite(scale)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_prefill: scale must be finite");
  }
  if (num_seqs == 0 || capacity == 0) return NKV_OK;
  if (!q || !key_cache || !value_cache || !out || !plan || !cu_seqlens_q || !cu_seqlens_k ||
      (table_stride > 0 && !block_tables)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_prefill: null pointer");
  }
  if ((reinterpret_cast<uint64_t>(q) | reinterpret_cast<uint64_t>(key_cache) |
       reinterpret_cast<uint64_t>(value_cache) | reinterpret_cast<uint64_t>(plan) |
       static_cast<uint64_t>(q_token_stride * 2)) % 16 != 0 ||
      (reinterpret_cast<uint64_t>(out) | static_cast<uint64_t>(out_token_stride * 2)) % 8 != 0) {
    return nkv_fail(NKV_E_INVALID,
                    "nkv_paged_attention_prefill: q/caches/plan must be 16-byte aligned and out "
                    "rows 8-byte aligned");
  }
  const float scale_log2 = scale * 1.4426950408889634f;  // log2(e)
  if (!(scale_log2 > 0.f)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_prefill: scale must be positive");
  }
  int32_t block_shift = -1;
  if ((block_size & (block_size - 1)) == 0) {
    block_shift = 0;
    while ((int64_t{1} << block_shift) < block_size) ++block_shift;
  }
  // Byte offsets of rows into one cache fit 32 bits unless the cache is
  // larger than 4 GiB; then the copies form 64-bit addresses.
  const int64_t row_bytes = num_kv_heads * head_dim * 2;
  const bool wide = num_blocks * block_size * row_bytes > static_cast<int64_t>(UINT32_MAX);
  const int64_t group = num_q_heads / num_kv_heads;
  const PrefillKernel kernel =
      half ? (wide ? prefill_kernel_for<true, true>(group)
                   : prefill_kernel_for<false, true>(group))
           : (wide ? prefill_kernel_for<true, false>(group)
                   : prefill_kernel_for<false, false>(group));
  int32_t xcd_layout = 0;
  int64_t grid = capacity * num_kv_heads;
  if (num_kv_heads % kXcds == 0) {
    xcd_layout = 1;
  } else if (kXcds % num_kv_heads == 0) {
    xcd_layout = 2;
    const int64_t per_head = kXcds / num_kv_heads;
    grid = kXcds * ((capacity + per_head - 1) / per_head);
  }
  if (grid > static_cast<int64_t>(UINT32_MAX / kPfThreads)) {
    return nkv_fail(NKV_E_INVALID, "nkv_paged_attention_prefill: %lld query tiles x %lld kv heads "
                    "exceed one launch", static_cast<long long>(capacity),
                    static_cast<long long>(num_kv_heads));
  }
  kernel<<<dim3(static_cast<unsigned>(grid)), dim3(kPfThreads), 0,
           static_cast<hipStream_t>(stream)>>>(
      static_cast<const uint16_t*>(q), q_token_stride, static_cast<const uint8_t*>(key_cache),
      static_cast<const uint8_t*>(value_cache), block_tables, table_stride,
      static_cast<int32_t>(block_size), block_shift, static_cast<int32_t>(num_blocks),
      static_cast<int32_t>(num_kv_heads), cu_seqlens_q, cu_seqlens_k,
      static_cast<const int4*>(plan), static_cast<int32_t>(capacity), xcd_layout,
      static_cast<int32_t>(num_seqs), scale_log2, static_cast<uint16_t*>(out), out_token_stride);
  return nkv_check_launch("nkv_paged_attention_prefill");
}
