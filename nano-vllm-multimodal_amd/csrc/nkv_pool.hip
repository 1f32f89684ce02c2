// Device block pool: the reference BlockManager's block bookkeeping — the
// free-block FIFO, the reference counts and the per-sequence block tables
// (nanovllm/engine/block_manager.py:87-118 _allocate_block /
// _deallocate_block, 185-236 allocate / deallocate / may_append) — kept in
// HBM and driven by an op log in the scheduler's call order, so the block
// tables the packer and the gather read never travel from the host.  The
// prefix-hash chain stays with the caller, which passes each allocation's
// cached-prefix block ids (what BlockManager.allocate re-derives from its
// hash map).
//
// State (one device buffer the caller owns, laid out by pool_layout):
//   ring[cap]   the free FIFO as a ring of cap = 2*num_blocks slots,
//               addressed by absolute positions [head, tail); a prefix hit
//               on a free block (the reference's free_block_ids.remove)
//               leaves a tombstone (-1) where the block stood, which pops
//               skip, so the remaining blocks keep their order;
//   qpos[NB]    absolute position of a free block's entry, -1 when used;
//   ref[NB]     reference counts;
//   tables[S*W] block table of each sequence slot, -1 padded; nblk[S].
//   meta        head, tail, live (free blocks), first error (op + 1, code).
// Tombstones plus re-freed blocks can make tail - head exceed num_blocks;
// when a push would overflow the ring, the live entries are compacted in
// order first.
//
// One workgroup of 1024 threads applies the whole log: ops are sequential
// (each depends on the queue the previous one left), the work inside an op
// is parallel (block-wide scans order the pops and pushes), and a run of
// appends, or of allocations without cached ids, to distinct slots is one
// parallel pop in op order.  Every op is validated before it changes
// anything; the first invalid op is recorded in meta and ends the log, so
// the state is always the reference's state after the valid prefix of the
// log.
#include "nkv_common.h"

namespace nkv {
namespace {

constexpr int kPoolThreads = 1024;
constexpr int kMetaWords = 8;  // head, tail, live, error op + 1, error code

struct PoolView {
  int64_t* meta;
  int32_t* ring;
  int64_t* qpos;
  int32_t* ref;
  int32_t* tables;
  int32_t* nblk;
  int32_t* slot_mark;  // scratch, zero between launches
  int32_t num_blocks;
  int32_t max_seqs;
  int32_t width;
  int64_t cap;
};

int64_t align256(int64_t n) { return (n + 255) & ~int64_t{255}; }

// Byte offsets of META, RING, QPOS, REF, TABLES, NBLK, the slot-mark
// scratch (int32[max_seqs], zero between launches) and the total size.
void pool_layout(int64_t num_blocks, int64_t max_seqs, int64_t width, int64_t offsets[8]) {
  const int64_t sizes[7] = {kMetaWords * 8, 2 * num_blocks * 4, num_blocks * 8, num_blocks * 4,
                            max_seqs * width * 4, max_seqs * 4, max_seqs * 4};
  int64_t at = 0;
  for (int k = 0; k < 7; ++k) {
    offsets[k] = at;
    at += align256(sizes[k]);
  }
  offsets[7] = at;
}

bool geometry_ok(int64_t num_blocks, int64_t max_seqs, int64_t width) {
  return num_blocks > 0 && num_blocks <= NKV_POOL_MAX_BLOCKS && max_seqs > 0 &&
         max_seqs <= NKV_POOL_MAX_SEQS && width > 0 && width <= num_blocks &&
         max_seqs * width <= INT32_MAX;
}

PoolView view_of(const nkv_pool_desc& d) {
  int64_t off[8];
  pool_layout(d.num_blocks, d.max_seqs, d.max_blocks_per_seq, off);
  auto* base = static_cast<uint8_t*>(d.memory);
  return PoolView{reinterpret_cast<int64_t*>(base + off[0]), reinterpret_cast<int32_t*>(base + off[1]),
                  reinterpret_cast<int64_t*>(base + off[2]), reinterpret_cast<int32_t*>(base + off[3]),
                  reinterpret_cast<int32_t*>(base + off[4]), reinterpret_cast<int32_t*>(base + off[5]),
                  reinterpret_cast<int32_t*>(base + off[6]),
                  static_cast<int32_t>(d.num_blocks), static_cast<int32_t>(d.max_seqs),
                  static_cast<int32_t>(d.max_blocks_per_seq), 2 * d.num_blocks};
}

__global__ void pool_init_kernel(PoolView v) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t start = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  for (int64_t i = start; i < v.cap; i += stride) {
    v.ring[i] = i < v.num_blocks ? static_cast<int32_t>(i) : -1;
  }
  for (int64_t i = start; i < v.num_blocks; i += stride) {
    v.qpos[i] = i;
    v.ref[i] = 0;
  }
  const int64_t cells = static_cast<int64_t>(v.max_seqs) * v.width;
  for (int64_t i = start; i < cells; i += stride) v.tables[i] = -1;
  for (int64_t i = start; i < v.max_seqs; i += stride) {
    v.nblk[i] = 0;
    v.slot_mark[i] = 0;
  }
  if (start == 0) {
    v.meta[0] = 0;             // head
    v.meta[1] = v.num_blocks;  // tail
    v.meta[2] = v.num_blocks;  // live
    for (int k = 3; k < kMetaWords; ++k) v.meta[k] = 0;
  }
}

// Block-wide sum of one value per thread (every thread gets the total).
__device__ __forceinline__ int32_t block_count(int32_t flag, int32_t* s_tmp) {
  int32_t total = 0;
  (void)block_exclusive_scan<kPoolThreads>(flag, s_tmp, &total);
  return total;
}

// The queue cursor, held identically by every thread (all updates derive
// from block-wide totals, so they stay uniform).
struct Cursor {
  int64_t head, tail, live;
};

// Rewrites the live entries of [head, tail) contiguously from head, in
// order (tombstones dropped).  Writes never pass the chunk being read, and
// the scan's barrier separates each chunk's reads from its writes.
__device__ void compact(const PoolView& v, Cursor& c, int32_t* s_tmp) {
  int64_t w = c.head;
  for (int64_t p = c.head; p < c.tail; p += kPoolThreads) {
    const int64_t q = p + threadIdx.x;
    const int32_t b = q < c.tail ? v.ring[q % v.cap] : -1;
    const int32_t live = b >= 0 ? 1 : 0;
    int32_t total = 0;
    const int32_t rank = block_exclusive_scan<kPoolThreads>(live, s_tmp, &total);
    if (live) {
      v.ring[(w + rank) % v.cap] = b;
      v.qpos[b] = w + rank;
    }
    w += total;
    __syncthreads();
  }
  c.tail = w;
}

// Takes the first m live entries from the front (the reference's popleft,
// tombstones skipped); sink(k, block) receives the k-th in order.  Requires
// c.live >= m.
template <typename Sink>
__device__ void pop_front(const PoolView& v, Cursor& c, int32_t m, int32_t* s_tmp,
                          int64_t* s_pos, Sink sink) {
  int32_t taken = 0;
  int64_t p = c.head;
  while (taken < m && p < c.tail) {
    const int64_t q = p + threadIdx.x;
    const int32_t b = q < c.tail ? v.ring[q % v.cap] : -1;
    const int32_t live = b >= 0 ? 1 : 0;
    int32_t total = 0;
    const int32_t rank = block_exclusive_scan<kPoolThreads>(live, s_tmp, &total);
    const int32_t need = m - taken;
    if (live && rank < need) {
      sink(taken + rank, b);
      v.qpos[b] = -1;
    }
    if (total >= need) {
      if (live && rank == need - 1) *s_pos = q + 1;
      __syncthreads();
      p = *s_pos;
      taken = m;
    } else {
      taken += total;
      p = min(p + kPoolThreads, c.tail);
    }
    __syncthreads();
  }
  c.head = p;
  c.live -= m;
}

enum : int32_t {
  kErrBadOp = NKV_POOL_ERR_BAD_OP,
  kErrBadSlot = NKV_POOL_ERR_BAD_SLOT,
  kErrTableBusy = NKV_POOL_ERR_TABLE_BUSY,
  kErrTableFull = NKV_POOL_ERR_TABLE_FULL,
  kErrNoFreeBlocks = NKV_POOL_ERR_NO_FREE,
  kErrBadBlock = NKV_POOL_ERR_BAD_BLOCK,
  kErrBadArgs = NKV_POOL_ERR_BAD_ARGS,
};

// The run of ops starting at i that `qualifies` (at most kPoolThreads of
// them), cut before the first op whose slot already appeared in the run, so
// the run's ops touch distinct tables and can proceed in parallel.  Slot
// marks (zero between launches) find the first occurrence of each slot:
// every op raises its slot's mark to kPoolThreads - k, so the mark names
// the smallest k.  Thread k returns ops[i + k] in *mine.
template <typename Qualifies>
__device__ int32_t run_length(const PoolView& v, const int4* __restrict__ ops, int64_t i,
                              int64_t num_ops, Qualifies qualifies, int32_t* s_end,
                              int4* mine) {
  const int32_t t = threadIdx.x;
  const int32_t n = static_cast<int32_t>(min<int64_t>(kPoolThreads, num_ops - i));
  if (t == 0) *s_end = n;
  __syncthreads();
  int4 op = make_int4(0, -1, 0, 0);
  if (t < n) {
    op = ops[i + t];
    if (!qualifies(op)) atomicMin(s_end, t);
  }
  *mine = op;
  __syncthreads();
  const int32_t end = *s_end;
  const bool marked = t < end && op.y >= 0 && op.y < v.max_seqs;
  if (marked) atomicMax(&v.slot_mark[op.y], kPoolThreads - t);
  __syncthreads();
  if (marked && __hip_atomic_load(&v.slot_mark[op.y], __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT) != kPoolThreads - t) {
    atomicMin(s_end, t);  // a repeat: the run stops before it
  }
  __syncthreads();
  if (marked) v.slot_mark[op.y] = 0;
  const int32_t cut = *s_end;
  __syncthreads();
  return cut;
}

// ops: int4 per op {type, slot, num_blocks (allocate), args offset
// (allocate)}; args[off] = number of cached ids, args[off+1 ...] the ids.
__global__ __launch_bounds__(kPoolThreads) void pool_apply_kernel(
    PoolView v, const int4* __restrict__ ops, int64_t num_ops,
    const int32_t* __restrict__ args, int64_t num_args) {
  __shared__ int32_t s_tmp[kPoolThreads / kWave + 1];
  __shared__ int32_t s_pre[kPoolThreads + 1];
  __shared__ int32_t s_slot[kPoolThreads];
  __shared__ int64_t s_pos;
  __shared__ int32_t s_end;
  __shared__ int32_t s_bad;
  const int32_t t = threadIdx.x;
  Cursor c{v.meta[0], v.meta[1], v.meta[2]};
  int32_t err = 0;
  int64_t err_op = 0;
  if (v.meta[4] != 0) return;  // an earlier log failed: the pool stays as it was

  int64_t i = 0;
  while (i < num_ops) {
    const int4 op = ops[i];
    if (op.x == NKV_POOL_OP_APPEND) {
      // A run of appends to distinct slots: one parallel pop for its valid
      // prefix; the first invalid op (or the first that finds no free
      // block) stops the log, as it would one op at a time.
      int4 mine;
      const int32_t run = run_length(
          v, ops, i, num_ops, [](const int4& o) { return o.x == NKV_POOL_OP_APPEND; }, &s_end,
          &mine);
      if (t == 0) s_bad = run;
      __syncthreads();
      int32_t code = 0;
      if (t < run) {
        if (mine.y < 0 || mine.y >= v.max_seqs) {
          code = kErrBadSlot;
        } else if (v.nblk[mine.y] >= v.width) {
          code = kErrTableFull;
        }
        if (code != 0) atomicMin(&s_bad, t);
      }
      __syncthreads();
      const int32_t first_bad = s_bad;
      if (t == first_bad && first_bad < run) s_bad = code;  // broadcast its code
      __syncthreads();
      const int32_t bad_code = first_bad < run ? s_bad : 0;
      const int32_t ok = static_cast<int32_t>(min<int64_t>(first_bad, c.live));
      if (t < ok) s_slot[t] = mine.y;
      __syncthreads();
      pop_front(v, c, ok, s_tmp, &s_pos, [&](int32_t k, int32_t b) {
        const int32_t slot = s_slot[k];
        const int32_t pos = v.nblk[slot];
        v.tables[static_cast<int64_t>(slot) * v.width + pos] = b;
        v.nblk[slot] = pos + 1;
        v.ref[b] = 1;
      });
      __syncthreads();
      if (ok < run) {
        err = ok == first_bad ? bad_code : kErrNoFreeBlocks;
        err_op = i + ok;
        break;
      }
      i += run;
      continue;
    }

    if (op.x == NKV_POOL_OP_ALLOCATE) {
      // A run of allocations without cached-prefix ids, to distinct slots:
      // the run's fresh blocks are one parallel pop in op order.
      int4 mine;
      const int32_t run = run_length(
          v, ops, i, num_ops,
          [&](const int4& o) {
            return o.x == NKV_POOL_OP_ALLOCATE && o.w >= 0 && o.w < num_args && args[o.w] == 0;
          },
          &s_end, &mine);
      if (run > 0) {
        if (t == 0) s_bad = run;
        __syncthreads();
        int32_t code = 0;
        if (t < run) {
          if (mine.y < 0 || mine.y >= v.max_seqs) {
            code = kErrBadSlot;
          } else if (v.nblk[mine.y] != 0) {
            code = kErrTableBusy;
          } else if (mine.z < 0 || mine.z > v.width) {
            code = kErrBadArgs;
          }
          if (code != 0) atomicMin(&s_bad, t);
        }
        __syncthreads();
        const int32_t first_bad = s_bad;
        if (t == first_bad && first_bad < run) s_bad = code;
        __syncthreads();
        const int32_t bad_code = first_bad < run ? s_bad : 0;
        // Fresh blocks needed up to each op, over the valid prefix.
        int32_t total = 0;
        const int32_t need = t < first_bad ? mine.z : 0;
        const int32_t before = block_exclusive_scan<kPoolThreads>(need, s_tmp, &total);
        if (t < run) {
          s_pre[t] = before;
          s_slot[t] = mine.y;
        }
        if (t == 0) s_end = first_bad;
        __syncthreads();
        // The first op whose blocks would not all be free.
        if (t < first_bad && before + need > c.live) atomicMin(&s_end, t);
        __syncthreads();
        const int32_t fits = s_end;
        const int32_t ok = min(first_bad, fits);
        if (t == 0) s_pre[ok] = ok < run ? s_pre[ok] : total;
        __syncthreads();
        const int32_t pops = s_pre[ok];
        pop_front(v, c, pops, s_tmp, &s_pos, [&](int32_t x, int32_t b) {
          const int32_t k = owner_of(s_pre, ok, x);
          v.tables[static_cast<int64_t>(s_slot[k]) * v.width + (x - s_pre[k])] = b;
          v.ref[b] = 1;
        });
        if (t < ok) v.nblk[s_slot[t]] = s_pre[t + 1] - s_pre[t];
        __syncthreads();
        if (ok < run) {
          err = ok == first_bad ? bad_code : kErrNoFreeBlocks;
          err_op = i + ok;
          break;
        }
        i += run;
        continue;
      }
    }

    if (op.x == NKV_POOL_OP_DEALLOCATE) {
      // A run of deallocations to distinct slots whose blocks are all held
      // once (no shared prefix): every block is freed, in op order and
      // reversed table order, so one pass places them all.  Anything else
      // (a shared or invalid block, a bad slot) takes the one-op path.
      int4 mine;
      const int32_t run = run_length(
          v, ops, i, num_ops, [](const int4& o) { return o.x == NKV_POOL_OP_DEALLOCATE; },
          &s_end, &mine);
      const bool slot_ok = t < run && mine.y >= 0 && mine.y < v.max_seqs;
      const int32_t n = slot_ok ? min(max(v.nblk[mine.y], 0), v.width) : 0;
      int32_t total = 0;
      const int32_t before = block_exclusive_scan<kPoolThreads>(n, s_tmp, &total);
      const int32_t bad_slots = block_count(t < run && !slot_ok ? 1 : 0, s_tmp);
      if (t < run) {
        s_pre[t] = before;
        s_slot[t] = mine.y;
      }
      if (t == 0) s_pre[run] = total;
      __syncthreads();
      int32_t unshared = 0;
      for (int32_t base = 0; base < total; base += kPoolThreads) {
        int32_t ok = 1;
        const int32_t x = base + t;
        if (x < total) {
          const int32_t k = owner_of(s_pre, run, x);
          const int32_t nk = s_pre[k + 1] - s_pre[k];
          const int32_t b =
              v.tables[static_cast<int64_t>(s_slot[k]) * v.width + (nk - 1 - (x - s_pre[k]))];
          ok = (b >= 0 && b < v.num_blocks && v.ref[b] == 1) ? 1 : 0;
        }
        unshared += block_count(ok, s_tmp);
      }
      if (bad_slots == 0 && unshared == (total + kPoolThreads - 1) / kPoolThreads * kPoolThreads) {
        if (c.tail - c.head + total > v.cap) compact(v, c, s_tmp);
        for (int32_t base = 0; base < total; base += kPoolThreads) {
          const int32_t x = base + t;
          if (x < total) {
            const int32_t k = owner_of(s_pre, run, x);
            const int32_t nk = s_pre[k + 1] - s_pre[k];
            int32_t* cell =
                v.tables + static_cast<int64_t>(s_slot[k]) * v.width + (nk - 1 - (x - s_pre[k]));
            const int32_t b = *cell;
            const int64_t pos = c.tail + x;
            v.ring[pos % v.cap] = b;
            v.qpos[b] = pos;
            v.ref[b] = 0;
            *cell = -1;
          }
        }
        if (t < run) v.nblk[mine.y] = 0;
        c.tail += total;
        c.live += total;
        __syncthreads();
        i += run;
        continue;
      }
    }

    const int32_t slot = op.y;
    if (slot < 0 || slot >= v.max_seqs) {
      err = kErrBadSlot;
      err_op = i;
      break;
    }
    int32_t* row = v.tables + static_cast<int64_t>(slot) * v.width;

    if (op.x == NKV_POOL_OP_ALLOCATE) {
      const int32_t n_total = op.z;
      const int64_t off = op.w;
      if (v.nblk[slot] != 0) {
        err = kErrTableBusy;
      } else if (n_total < 0 || n_total > v.width || off < 0 || off >= num_args) {
        err = kErrBadArgs;
      } else {
        const int32_t n_cached = args[off];
        if (n_cached < 0 || n_cached > n_total || off + 1 + n_cached > num_args) err = kErrBadArgs;
      }
      if (err != 0) {
        err_op = i;
        break;
      }
      const int32_t n_cached = args[off];
      const int32_t* cached = args + off + 1;
      // Validate every cached id and count the free ones (they leave the
      // queue) before touching anything.
      int32_t bad = 0, hits_free = 0;
      for (int32_t base = 0; base < n_cached; base += kPoolThreads) {
        int32_t my_bad = 0, my_free = 0;
        if (base + t < n_cached) {
          const int32_t b = cached[base + t];
          if (b < 0 || b >= v.num_blocks) {
            my_bad = 1;
          } else if (v.ref[b] == 0) {
            my_free = 1;
          }
        }
        bad += block_count(my_bad, s_tmp);
        hits_free += block_count(my_free, s_tmp);
      }
      if (bad != 0 || c.live - hits_free < n_total - n_cached) {
        err = bad != 0 ? kErrBadBlock : kErrNoFreeBlocks;
        err_op = i;
        break;
      }
      for (int32_t base = 0; base < n_cached; base += kPoolThreads) {
        if (base + t < n_cached) {
          const int32_t b = cached[base + t];
          if (v.ref[b] > 0) {
            v.ref[b] += 1;
          } else {
            v.ref[b] = 1;
            const int64_t qp = v.qpos[b];
            if (qp >= 0) v.ring[qp % v.cap] = -1;  // leaves the queue where it stands
            v.qpos[b] = -1;
          }
          row[base + t] = b;
        }
      }
      c.live -= hits_free;
      __syncthreads();
      pop_front(v, c, n_total - n_cached, s_tmp, &s_pos, [&](int32_t k, int32_t b) {
        row[n_cached + k] = b;
        v.ref[b] = 1;
      });
      if (t == 0) v.nblk[slot] = n_total;
      __syncthreads();
      ++i;
      continue;
    }

    if (op.x == NKV_POOL_OP_DEALLOCATE) {
      const int32_t n = min(max(v.nblk[slot], 0), v.width);
      int32_t bad = 0;
      for (int32_t base = 0; base < n; base += kPoolThreads) {
        int32_t my_bad = 0;
        if (base + t < n) {
          const int32_t b = row[base + t];
          my_bad = (b < 0 || b >= v.num_blocks || v.ref[b] <= 0) ? 1 : 0;
        }
        bad += block_count(my_bad, s_tmp);
      }
      if (bad != 0) {
        err = kErrBadBlock;
        err_op = i;
        break;
      }
      if (c.tail - c.head + n > v.cap) compact(v, c, s_tmp);
      // Reversed table order; a block whose count reaches zero goes to the
      // back of the queue, in that order.
      for (int32_t base = 0; base < n; base += kPoolThreads) {
        const int32_t r = base + t;
        int32_t freed = 0, b = -1;
        if (r < n) {
          b = row[n - 1 - r];
          const int32_t left = v.ref[b] - 1;
          v.ref[b] = left;
          freed = left == 0 ? 1 : 0;
          row[n - 1 - r] = -1;
        }
        int32_t total = 0;
        const int32_t rank = block_exclusive_scan<kPoolThreads>(freed, s_tmp, &total);
        if (freed) {
          const int64_t pos = c.tail + rank;
          v.ring[pos % v.cap] = b;
          v.qpos[b] = pos;
        }
        c.tail += total;
        c.live += total;
      }
      if (t == 0) v.nblk[slot] = 0;
      __syncthreads();
      ++i;
      continue;
    }

    if (op.x != NKV_POOL_OP_FENCE) {
      err = kErrBadOp;
      err_op = i;
      break;
    }
    ++i;
  }
  if (t == 0) {
    v.meta[0] = c.head;
    v.meta[1] = c.tail;
    v.meta[2] = c.live;
    if (err != 0) {
      v.meta[3] = err_op + 1;
      v.meta[4] = err;
    }
  }
}

// Rejects descriptors the kernels could not use safely.
int check_desc(const nkv_pool_desc* d, const char* what) {
  if (d == nullptr || d->memory == nullptr) return nkv_fail(NKV_E_INVALID, "%s: null pool", what);
  if (!geometry_ok(d->num_blocks, d->max_seqs, d->max_blocks_per_seq)) {
    return nkv_fail(NKV_E_INVALID,
                    "%s: need 0 < num_blocks <= %d, 0 < max_seqs <= %d, "
                    "0 < max_blocks_per_seq <= num_blocks",
                    what, NKV_POOL_MAX_BLOCKS, NKV_POOL_MAX_SEQS);
  }
  if (reinterpret_cast<uint64_t>(d->memory) % 256 != 0) {
    return nkv_fail(NKV_E_INVALID, "%s: pool memory must be 256-byte aligned", what);
  }
  return NKV_OK;
}

}  // namespace
}  // namespace nkv

extern "C" int64_t nkv_pool_bytes(int64_t num_blocks, int64_t max_seqs,
                                  int64_t max_blocks_per_seq) {
  if (!nkv::geometry_ok(num_blocks, max_seqs, max_blocks_per_seq)) return 0;
  int64_t off[8];
  nkv::pool_layout(num_blocks, max_seqs, max_blocks_per_seq, off);
  return off[7];
}

extern "C" int nkv_pool_offsets(int64_t num_blocks, int64_t max_seqs,
                                int64_t max_blocks_per_seq, int64_t* offsets) {
  if (offsets == nullptr) return nkv_fail(NKV_E_INVALID, "nkv_pool_offsets: null output");
  if (!nkv::geometry_ok(num_blocks, max_seqs, max_blocks_per_seq)) {
    return nkv_fail(NKV_E_INVALID, "nkv_pool_offsets: bad geometry");
  }
  int64_t off[8];
  nkv::pool_layout(num_blocks, max_seqs, max_blocks_per_seq, off);
  for (int k = 0; k < 6; ++k) offsets[k] = off[k];
  return NKV_OK;
}

extern "C" int nkv_pool_init(const nkv_pool_desc* pool, void* stream) {
  using namespace nkv;
  if (int rc = check_desc(pool, "nkv_pool_init")) return rc;
  pool_init_kernel<<<dim3(256), dim3(256), 0, static_cast<hipStream_t>(stream)>>>(view_of(*pool));
  return nkv_check_launch("nkv_pool_init");
}

extern "C" int nkv_pool_apply(const nkv_pool_desc* pool, const int32_t* ops, int64_t num_ops,
                              const int32_t* args, int64_t num_args, void* stream) {
  using namespace nkv;
  if (int rc = check_desc(pool, "nkv_pool_apply")) return rc;
  if (num_ops < 0 || num_args < 0 || num_ops > INT32_MAX || num_args > INT32_MAX) {
    return nkv_fail(NKV_E_INVALID, "nkv_pool_apply: negative or oversized op log");
  }
  if (num_ops == 0) return NKV_OK;
  if (ops == nullptr || (num_args > 0 && args == nullptr)) {
    return nkv_fail(NKV_E_INVALID, "nkv_pool_apply: null pointer");
  }
  if (reinterpret_cast<uint64_t>(ops) % 16 != 0) {
    return nkv_fail(NKV_E_INVALID, "nkv_pool_apply: ops must be 16-byte aligned");
  }
  pool_apply_kernel<<<dim3(1), dim3(kPoolThreads), 0, static_cast<hipStream_t>(stream)>>>(
      view_of(*pool), reinterpret_cast<const int4*>(ops), num_ops, args, num_args);
  return nkv_check_launch("nkv_pool_apply");
}

namespace nkv {

int pool_tables(const nkv_pool_desc* pool, const char* what, const int32_t** tables,
                const int32_t** nblk) {
  if (int rc = check_desc(pool, what)) return rc;
  const PoolView v = view_of(*pool);
  *tables = v.tables;
  *nblk = v.nblk;
  return NKV_OK;
}

}  // namespace nkv
