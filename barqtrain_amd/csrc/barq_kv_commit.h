// Launch-internal commit of an append, shared by the kernels that fuse an append with other work
// (barq_kv.hip's stream kernels, barq_kv_quant.hip's dequantising update): wave-wide scans on
// DPP, the new-block rule, and the arrival counters whose last arrival maps the new blocks and
// advances the rows.  Device code only; every function is inline.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>

#include "barq_kv.h"
#include "fastdiv.h"

namespace barq_commit {

constexpr int kWave = 64;

__device__ __forceinline__ int ceil_div_fd(int n, const FastDiv& d) {
  return n <= 0 ? 0 : (int)d.div((uint32_t)(n + (int)d.d - 1));
}

// A page id read from the stack or the table, or -1 when it names no page of the pool.
__device__ __forceinline__ int checked_page(int page, int64_t num_pages) {
  return (page >= 0 && (int64_t)page < num_pages) ? page : -1;
}

// Wave-wide inclusive scan on DPP: row shifts by 1, 2, 4, 8 scan each 16-lane row, then the
// row broadcasts of lanes 15 and 31 carry row totals into rows 1, 3 and 2, 3.  Each step is a
// VALU operation on register data; the ds_bpermute that a shuffle compiles to costs an LDS
// round trip per step, and the control wave runs these on every launch's critical path.
// Lanes a shift or broadcast does not reach keep `identity`.  The whole wave must be active.
struct AddOp {
  __device__ int operator()(int a, int b) const { return a + b; }
};
struct MaxOp {
  __device__ int operator()(int a, int b) const { return max(a, b); }
};

template <typename Op>
__device__ __forceinline__ int wave_scan_dpp(int v, int identity, Op op) {
  v = op(v, __builtin_amdgcn_update_dpp(identity, v, 0x111, 0xf, 0xf, false));  // row_shr:1
  v = op(v, __builtin_amdgcn_update_dpp(identity, v, 0x112, 0xf, 0xf, false));  // row_shr:2
  v = op(v, __builtin_amdgcn_update_dpp(identity, v, 0x114, 0xf, 0xf, false));  // row_shr:4
  v = op(v, __builtin_amdgcn_update_dpp(identity, v, 0x118, 0xf, 0xf, false));  // row_shr:8
  v = op(v, __builtin_amdgcn_update_dpp(identity, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
  v = op(v, __builtin_amdgcn_update_dpp(identity, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
  return v;
}

// Sum / maximum over the wave, uniform (returned in a scalar register).
__device__ __forceinline__ int wave_sum(int v) {
  return __builtin_amdgcn_readlane(wave_scan_dpp(v, 0, AddOp()), kWave - 1);
}

__device__ __forceinline__ int wave_max(int v) {
  return __builtin_amdgcn_readlane(wave_scan_dpp(v, INT_MIN, MaxOp()), kWave - 1);
}

__device__ __forceinline__ int wave_incl_scan(int v) { return wave_scan_dpp(v, 0, AddOp()); }

// Number of blocks of a row that an append of `tokens` maps for the first time, and the first
// of them.  Blocks at or beyond max_blocks are never mapped (the capacity bit reports them).
struct NewBlocks {
  int first;
  int count;
};

__device__ __forceinline__ NewBlocks new_blocks(int len, int hw, int tokens, int max_blocks,
                                                const FastDiv& div_page) {
  NewBlocks nb;
  nb.first = ceil_div_fd(hw, div_page);
  const int end = min(ceil_div_fd(len + tokens, div_page), max_blocks);
  nb.count = tokens > 0 ? max(0, end - nb.first) : 0;
  return nb;
}

// The same commit by one wave, from metadata its lanes already hold (batch <= kWave): lane r
// holds row r's length and high-water mark, lane k holds free_pages[top - 1 - k], the page the
// k-th new block takes.  The new blocks are mapped one rank per lane, 64 ranks a round; ranks
// past the first 64 read their page from the stack, eight rounds' reads in flight at once.
__device__ inline void commit_from_lanes(const barq_kv_pool& p, int batch, int tokens, int limit,
                                  const FastDiv& div_page, int len, int hw, int top, int free_k) {
  const int lane = threadIdx.x & (kWave - 1);
  const int mb = (int)p.max_blocks;
  int err = 0;
  NewBlocks nb{0, 0};
  if (lane < batch) {
    nb = new_blocks(len, hw, tokens, mb, div_page);
    if (ceil_div_fd(len + tokens, div_page) > mb) err |= BARQ_KV_ERRBIT_CAPACITY;
    if (len + tokens > limit) err |= BARQ_KV_ERRBIT_OUT_SHORT;
  }
  const int incl = wave_incl_scan(nb.count);
  const int total = __builtin_amdgcn_readlane(incl, kWave - 1);
  constexpr int kGroup = 8;  // 64-rank rounds whose stack reads are in flight together
  for (int g0 = 0; g0 < total; g0 += kGroup * kWave) {
    int pg[kGroup];
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int k = g0 + u * kWave + lane;
      const int idx = top - 1 - k;
      pg[u] = -1;
      if (k < total && idx >= 0) pg[u] = (g0 == 0 && u == 0) ? free_k : p.free_pages[idx];
    }
#pragma unroll
    for (int u = 0; u < kGroup; ++u) {
      const int k0 = g0 + u * kWave;
      if (k0 >= total) break;
      const int k = k0 + lane;
      // Rank k belongs to row `row`: the number of rows whose rank end is at most k.
      int row = 0;
      for (int r = 0; r < batch; ++r) row += k >= __builtin_amdgcn_readlane(incl, r) ? 1 : 0;
      const int src = row & (kWave - 1);
      const int row_first = __shfl(nb.first, src, kWave);
      const int row_excl = __shfl(incl - nb.count, src, kWave);
      if (k < total) {
        const int page = top - 1 - k >= 0 ? checked_page(pg[u], p.num_pages) : -1;
        if (page < 0) err |= BARQ_KV_ERRBIT_POOL_EXHAUSTED;
        p.block_table[(int64_t)row * mb + row_first + (k - row_excl)] = page;
      }
    }
  }
  if (lane < batch) {
    p.seq_lens[lane] = len + tokens;
    p.high_water[lane] = max(hw, len + tokens);
  }
  if (lane == 0) p.ctrl[BARQ_KV_CTRL_FREE_TOP] = max(0, top - total);
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// The tile arrives -- on one of BARQ_KV_CTRL_SUBCOUNTERS sub-counters, whose last arrivals count
// on the main counter -- and the last tile to arrive commits the launch's append.  A
// sub-counter's last arrival reads the commit inputs (every row's length and mark, the stack
// top) together with its main arrival: until the last arrival commits nothing writes them, so
// they are the launch's starting state.  The stack entries new blocks take are read only when
// there are new blocks.  Run by a whole wave (the control wave), after every wave of the tile
// holds the metadata it uses.
__device__ inline void arrive_and_commit(const barq_kv_pool& p, int nsub, int batch, int tokens, int limit,
                                  const FastDiv& div_page) {
  const int lane = threadIdx.x & (kWave - 1);
  int sublast = 0;
  if (lane == 0) {
    const int sub = (int)blockIdx.x % nsub;
    const int expect = ((int)gridDim.x - sub + nsub - 1) / nsub;
    int* counter = &p.ctrl[BARQ_KV_CTRL_SUBCOUNTER0 + sub * BARQ_KV_CTRL_SUBCOUNTER_STRIDE];
    sublast = atomicAdd(counter, 1) == expect - 1;
    if (sublast) atomicExch(counter, 0);
  }
  if (!__builtin_amdgcn_readfirstlane(sublast)) return;
  int last = 0;
  if (lane == 0) last = atomicAdd(&p.ctrl[BARQ_KV_CTRL_ARRIVED], 1) == nsub - 1;
  int c_len = 0, c_hw = 0;
  if (lane < batch) {
    c_len = p.seq_lens[lane];
    c_hw = p.high_water[lane];
  }
  const int c_top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
  if (!__builtin_amdgcn_readfirstlane(last)) return;
  const int news = wave_sum(lane < batch ? new_blocks(c_len, c_hw, tokens, (int)p.max_blocks, div_page).count : 0);
  const int fidx = c_top - 1 - lane;
  const int c_free = news > 0 && fidx >= 0 ? p.free_pages[fidx] : -1;
  commit_from_lanes(p, batch, tokens, limit, div_page, c_len, c_hw, c_top, c_free);
  if (lane == 0) atomicExch(&p.ctrl[BARQ_KV_CTRL_ARRIVED], 0);
}

}  // namespace barq_commit
