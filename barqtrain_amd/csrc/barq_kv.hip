// Paged KV-cache kernels for MI355X (gfx950) behind the C ABI of include/barq_kv.h.
//
// Storage of one layer: key/value pages [num_pages, page_size, kv_heads, head_dim], so one
// token's K (or V) across all heads is one contiguous run of kv_heads*head_dim elements -- the
// same run HF attention produces ([B, T, H, D] physical, viewed as [B, H, T, D]).  Rows reach
// their pages through an int32 block table; free pages sit on an int32 stack.  All element
// traffic is a bit copy, done in the widest vector (16, 8, 4, 2 or 1 bytes) that every
// address and stride admits.
//
// Semantics follow the reference layer (python/barqtrain/kv_cache.py:75-91,120-133): token t
// of row b is stored at slot seq_lens[b] + t, and a gathered slot s of row b is the value last
// stored there when s < high_water[b], else zero (the reference cache is zero-initialised,
// kv_cache.py:66-71, and crop() lowers seq_lens without clearing, :158-164).
//
// Page allocation is deterministic: the new blocks of a launch are ranked in (row, block)
// order and rank k takes free_pages[top - 1 - k].  Every tile can therefore compute the page
// of any new block on its own; the stack top, block table and row lengths are committed once
// per launch, inside the launch by the last tile to have read its metadata (arrival counters),
// or by a one-workgroup launch.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <climits>

#include "barq_kv.h"
#include "barq_kv_commit.h"
#include "fastdiv.h"

namespace {

using barq_commit::arrive_and_commit;
using barq_commit::ceil_div_fd;
using barq_commit::checked_page;
using barq_commit::commit_from_lanes;
using barq_commit::new_blocks;
using barq_commit::NewBlocks;
using barq_commit::wave_incl_scan;
using barq_commit::wave_max;
using barq_commit::wave_sum;

constexpr int kThreads = 256;                     // workgroup of the bookkeeping kernels
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kStreamThreads = kThreads + kWave;  // stream kernel: control wave + 4 copy waves
constexpr int kCopyWaves = kStreamThreads / kWave - 1;
constexpr int kUnroll = 16;                       // vectors in flight per copy thread
constexpr int kMaxTilePages = 64;                 // block-table slots a tile stages in LDS
// Positions per tile: whole pages, about this many bytes of K (or V).  With kUnroll 16-byte
// vectors per thread, a 64 KiB tile is loaded by the 256 copy threads in one batch.
constexpr int kTileTargetBytes = 64 * 1024;
// A launch of more tiles than this (about 1.5x the stream kernel's workgroups resident on the
// chip at once) takes tiles of half as many pages: once tiles run in several dispatch rounds,
// smaller tiles stream faster (bf16 8x128 heads, 32 KiB pages: 1.07 GB per launch 193 -> 179 us,
// 268 MB 53.4 -> 50.9 us), while a launch that is resident at once streams best from the
// larger tiles (84 MB: 16.6 us at 64 KiB, 18.4 us at 32 KiB; ~1000 tiles: even).
constexpr int64_t kLargeLaunchTiles = 1536;
// Stream-kernel tiles (five-wave workgroups) resident on one CU at once.
constexpr int64_t kResidentTilesPerCU = 4;

template <int VB>
struct VecT;
template <>
struct VecT<16> { using T = uint32_t __attribute__((ext_vector_type(4))); };
template <>
struct VecT<8> { using T = uint32_t __attribute__((ext_vector_type(2))); };
template <>
struct VecT<4> { using T = uint32_t; };
template <>
struct VecT<2> { using T = uint16_t; };
template <>
struct VecT<1> { using T = uint8_t; };

template <typename T>
__device__ __forceinline__ T zero_vec() { return T(0); }

// s_waitcnt with vmcnt = K (K < 16) and no wait on the other counters (gfx9 encoding: vmcnt
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int K>
__device__ __forceinline__ void wait_vm() {
  static_assert(K >= 0 && K < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(K | (0x7 << 4) | (0xF << 8));
}

// Streaming accesses (page reads, input reads, output writes): every byte is touched once per
// launch, so they carry the nontemporal hint and do not displace other data from the caches.
template <typename T>
__device__ __forceinline__ T ld_stream(const char* ptr) {
  return __builtin_nontemporal_load((const T*)ptr);
}
template <typename T>
__device__ __forceinline__ void st_stream(char* ptr, T v) {
  __builtin_nontemporal_store(v, (T*)ptr);
}

// Exclusive prefix sum of v over the workgroup's NW waves; *total gets the sum of all.
// Uses lds[0 .. NW).  Every thread of the workgroup must call it.
template <int NW>
__device__ __forceinline__ int block_exclusive_scan(int v, int* lds, int* total) {
  const int wave = threadIdx.x / kWave;
  const int incl = wave_incl_scan(v);
  if ((threadIdx.x & (kWave - 1)) == kWave - 1) lds[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const int t = lds[w];
    if (w < wave) before += t;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + incl - v;
}

// Rank of the first new block of row `row`: the number of new blocks of rows [0, row).
// Called by one whole wave.
__device__ int wave_rank_base(const barq_kv_pool& p, int row, int tokens,
                              const FastDiv& div_page) {
  const int lane = threadIdx.x & (kWave - 1);
  int acc = 0;
  for (int r0 = 0; r0 < row; r0 += kWave) {
    const int r = r0 + lane;
    int c = 0;
    if (r < row) c = new_blocks(p.seq_lens[r], p.high_water[r], tokens, (int)p.max_blocks, div_page).count;
    acc += wave_sum(c);
  }
  return acc;
}

// Commit an append of `tokens` to rows [0, batch): map new blocks to pages in rank order,
// advance seq_lens and high_water, pop the stack.  `limit` is the end of the positions the
// launch covered (an update covers its output extent only); a row whose new end passes it lost
// tokens and raises the OUT_SHORT bit.  Run by a whole workgroup of NTHREADS threads, after
// every tile that reads the old metadata has read it.
template <int NTHREADS>
__device__ void commit_append(const barq_kv_pool& p, int batch, int tokens, int limit,
                              const FastDiv& div_page) {
  __shared__ int lds_scan[NTHREADS / kWave];
  __shared__ int s_incl[NTHREADS];   // rank end of each row of the chunk
  __shared__ int s_first[NTHREADS];  // first new block of each row of the chunk
  const int top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
  const int mb = (int)p.max_blocks;
  const int tid = (int)threadIdx.x;
  int used = 0;
  int err = 0;
  for (int r0 = 0; r0 < batch; r0 += NTHREADS) {
    const int r = r0 + tid;
    int len = 0, hw = 0;
    NewBlocks nb{0, 0};
    if (r < batch) {
      len = p.seq_lens[r];
      hw = p.high_water[r];
      nb = new_blocks(len, hw, tokens, mb, div_page);
      if (ceil_div_fd(len + tokens, div_page) > mb) err |= BARQ_KV_ERRBIT_CAPACITY;
      if (len + tokens > limit) err |= BARQ_KV_ERRBIT_OUT_SHORT;
    }
    int chunk_total = 0;
    const int excl = block_exclusive_scan<NTHREADS / kWave>(nb.count, lds_scan, &chunk_total);
    s_incl[tid] = excl + nb.count;
    s_first[tid] = nb.first;
    __syncthreads();
    // The chunk's new blocks in rank order, one per thread: rank k belongs to the first row whose
    // rank end passes k, and takes free_pages[top - 1 - (used + k)].
    for (int k0 = 0; k0 < chunk_total; k0 += NTHREADS) {
      const int k = k0 + tid;
      if (k < chunk_total) {
        int lo = 0, hi = NTHREADS - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (s_incl[mid] > k) hi = mid;
          else lo = mid + 1;
        }
        const int row_excl = lo > 0 ? s_incl[lo - 1] : 0;
        const int idx = top - 1 - (used + k);
        const int page = idx >= 0 ? checked_page(p.free_pages[idx], p.num_pages) : -1;
        if (page < 0) err |= BARQ_KV_ERRBIT_POOL_EXHAUSTED;
        p.block_table[(int64_t)(r0 + lo) * mb + s_first[lo] + (k - row_excl)] = page;
      }
    }
    if (r < batch) {
      p.seq_lens[r] = len + tokens;
      p.high_water[r] = max(hw, len + tokens);
    }
    used += chunk_total;
    __syncthreads();  // s_incl / s_first are rewritten by the next chunk of rows
  }
  if (tid == 0) p.ctrl[BARQ_KV_CTRL_FREE_TOP] = max(0, top - used);
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// ---------------------------------------------------------------------------------------------
// Append / gather / update.
//
// One workgroup = one tile = (K or V, row, chunk of positions); a gather's chunks are whole
// pages.  Wave 0 is the control wave: it reads the tile's metadata (the row's length and mark,
// its block-table slice, the pages that new blocks take) into LDS.  After the barrier the copy
// waves 1..4 stream the tile, while the control wave counts the tile as arrived and, in the
// last tile to arrive, commits the append: every tile has read the old metadata by then, so the
// commit overlaps the copies instead of trailing them.  Arrivals go to BARQ_KV_CTRL_SUBCOUNTERS
// counters on separate 256-byte lines (tile i to counter i % nsub), whose last arrivals count
// on the main counter: a single counter hit by every tile at once serialises them.
// ---------------------------------------------------------------------------------------------

struct StreamArgs {
  barq_kv_pool pool;
  const char* in_k;
  const char* in_v;
  char* out_k;
  char* out_v;
  int64_t in_sb, in_sh, in_st;     // bytes
  int64_t out_sb, out_sh, out_ss;  // bytes
  int64_t page_bytes;
  int64_t tok_bytes;
  int32_t batch;
  int32_t tokens;
  int32_t seq_out;   // gather: positions covered by the grid (capacity with SEQ_FROM_DEVICE)
  int32_t chunk;     // positions per tile (pages_per_tile * page_size)
  int32_t ppt;       // pages per tile
  int32_t gather;    // write the materialised output
  int32_t seq_from_device;
  int32_t commit_in_kernel;  // the launch commits its own append
  int32_t hv;        // vectors per token (kv_heads * vr)
  int32_t nsub;      // arrival sub-counters in use
  int32_t full_tiles;  // tiles of `chunk` positions; the blocks after them are tail pieces
  int32_t tail_lo;     // gather: first position of the tail
  int32_t piece_len;   // gather: positions per tail piece
  FastDiv div_hv;    // by hv
  FastDiv div_vr;    // by vectors per head row
  FastDiv div_page;  // by page_size
  FastDiv div_chunks;
  FastDiv div_pieces;  // by tail pieces per (row, K or V)
};

// LPP > 0: hv = 64 * LPP (LPP = 1, 2 or 4) and offsets within a page, a row's output and a row's
// input fit 32 bits.  A copy wave then moves whole positions, 64 vectors per load, so position,
// block, page and output row are wave-uniform (scalar registers) and a lane's addresses differ
// only by its column offset.  LPP = 0: any geometry.
template <int VB, int LPP, bool ROUNDS>
__device__ __forceinline__ void stream_body(const StreamArgs& a) {
  using V = typename VecT<VB>::T;
  __shared__ int64_t s_pbase[kMaxTilePages + 1];  // byte offset of each block's page, or -1
  __shared__ int s_meta[6];                       // len, hw, lo, hi, blk_lo, last

  const barq_kv_pool& p = a.pool;
  // Block -> tile.  Blocks [0, full_tiles) are (K or V, row, chunk) tiles of `chunk` positions;
  // a gather launch may follow them with tail pieces, (K or V, row, piece) of piece_len
  // positions from tail_lo on, sized so that every CU receives the same work.
  const int bid = (int)blockIdx.x;
  const bool tail = bid >= a.full_tiles;
  int kv, b, c;
  if (!tail) {
    kv = bid & 1;
    const int rest = bid >> 1;
    b = (int)a.div_chunks.div((uint32_t)rest);
    c = rest - b * (int)a.div_chunks.d;
  } else {
    // Piece j of the tail: stream j / n, piece j mod n (n pieces per stream).
    const int j = bid - a.full_tiles;
    const int sid = (int)a.div_pieces.div((uint32_t)j);
    c = j - sid * (int)a.div_pieces.d;
    kv = sid & 1;
    b = sid >> 1;
  }
  const int tlo = tail ? a.tail_lo + c * a.piece_len : c * a.chunk;
  const int tlen = tail ? a.piece_len : a.chunk;
  const int T = a.tokens;
  const int P = (int)p.page_size;
  const int mb = (int)p.max_blocks;
  const bool committing = T > 0 && a.commit_in_kernel;
  const bool rows_in_lanes = a.batch <= kWave;
  // Early commit: the commit inputs (every row's length and mark, the stack top) sit in the
  // control wave's lanes, one row per lane.
  const bool early = committing && rows_in_lanes;

  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    // One round of independent loads: this row's length and mark (uniform: scalar cache) and the
    // tile's block-table slice (gather tiles are block aligned).  Batch-wide values -- the longest
    // row, the rank of this row's new blocks -- are read only by the tiles that need them: every
    // tile reading the same lines of seq_lens / high_water at once serialises those reads on one
    // L2 channel (at C2 about 1.5 us of a 15 us launch).
    const int len = p.seq_lens[b];
    const int hw = p.high_water[b];
    int pre = -1;
    const int gb0 = (int)a.div_page.div((uint32_t)tlo);  // first block of a gather tile
    if (a.gather && lane <= a.ppt && gb0 + lane < mb) pre = p.block_table[(int64_t)b * mb + gb0 + lane];
    int rl = 0, rh = 0;  // lane r < batch: row r's length and mark, once loaded
    bool rows_loaded = false;
    int smax = a.seq_out;
    // A gather tile reaching past its own row's end (capped by the buffer) needs the longest row.
    if (a.gather && a.seq_from_device && tlo + tlen > min(len + T, a.seq_out)) {
      int m = 0;
      if (rows_in_lanes) {
        if (lane < a.batch) {
          rl = p.seq_lens[lane];
          rh = p.high_water[lane];
          m = rl + T;
        }
        rows_loaded = true;
      } else {
        for (int r = lane; r < a.batch; r += kWave) m = max(m, p.seq_lens[r] + T);
      }
      smax = min(wave_max(m), a.seq_out);
    }
    int lo, hi;
    if (a.gather) {
      lo = tlo;
      hi = min(lo + tlen, smax);
    } else {
      lo = len + c * a.chunk;
      hi = min(lo + a.chunk, len + T);
    }
    int blk_lo = 0, nblk = 0;
    if (hi > lo) {
      blk_lo = (int)a.div_page.div((uint32_t)lo);
      nblk = (int)a.div_page.div((uint32_t)(hi - 1)) - blk_lo + 1;
    }
    const NewBlocks nb = new_blocks(len, hw, T, mb, a.div_page);
    const bool touches_new = nb.count > 0 && blk_lo < nb.first + nb.count && blk_lo + nblk > nb.first;
    int base = 0, top = 0;
    if (touches_new) {
      top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
      if (rows_in_lanes) {
        if (!rows_loaded && lane < a.batch) {
          rl = p.seq_lens[lane];
          rh = p.high_water[lane];
        }
        base = wave_sum(lane < b ? new_blocks(rl, rh, T, mb, a.div_page).count : 0);
      } else {
        base = wave_rank_base(p, b, T, a.div_page);
      }
    }
    // nblk <= kMaxTilePages + 1 (an append chunk may start mid-block): two slots per lane.
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int i = lane + k * kWave;
      if (i < nblk) {
        const int blk = blk_lo + i;
        int page = -1;
        if (blk < mb) {
          if (blk < nb.first) {
            page = checked_page((a.gather && k == 0) ? pre : p.block_table[(int64_t)b * mb + blk], p.num_pages);
          } else if (blk < nb.first + nb.count) {
            const int idx = top - 1 - (base + blk - nb.first);
            page = idx >= 0 ? checked_page(p.free_pages[idx], p.num_pages) : -1;
          }
        }
        s_pbase[i] = page >= 0 ? (int64_t)page * a.page_bytes : (int64_t)-1;
      }
    }
    if (lane == 0) {
      s_meta[0] = len;
      s_meta[1] = hw;
      s_meta[2] = lo;
      s_meta[3] = hi;
      s_meta[4] = blk_lo;
    }
  }
  __syncthreads();

  if (early && threadIdx.x < kWave) {
    // Control wave.  Every metadata value this tile uses was read before the barrier, so the
    // tile arrives now, and the copy waves never wait for the arrival or the commit.
    arrive_and_commit(p, a.nsub, a.batch, T, a.gather ? a.seq_out : INT_MAX, a.div_page);
    return;
  }

  const int len = s_meta[0];
  const int hw = s_meta[1];
  const int lo = s_meta[2];
  const int hi = s_meta[3];
  const int blk_lo = s_meta[4];
  const int npos = hi > lo ? hi - lo : 0;

  const char* in = kv ? a.in_v : a.in_k;
  char* pages = (char*)(kv ? p.value_pages : p.key_pages);
  char* out = kv ? a.out_v : a.out_k;
  const int wave = (int)(threadIdx.x / kWave);

  if constexpr (LPP > 0 && ROUNDS) {
    // Launches whose tiles run in several rounds.  Same wave mapping as below; each load's page
    // comes from LDS just before it is issued and stores wait for the previous one, which spaces
    // a wave's requests.  Measured best once tiles start at different times (C4 0.62 of HBM peak
    // against 0.57 with back-to-back loads; C5 0.72 against 0.69).
    constexpr int RSTEP = 4 / LPP;
    if (wave > 0) {
      const int lane = (int)(threadIdx.x & (kWave - 1));
      const int r0 = __builtin_amdgcn_readfirstlane((wave - 1) / LPP);
      const int col = ((wave - 1) % LPP) * kWave + lane;
      const int h = (int)a.div_vr.div((uint32_t)col);
      const int v = col - h * (int)a.div_vr.d;
      const uint32_t page_lane = (uint32_t)(col * VB);
      const uint32_t out_lane = (uint32_t)((int64_t)h * a.out_sh + (int64_t)v * VB);
      const uint32_t in_lane = (uint32_t)((int64_t)h * a.in_sh + (int64_t)v * VB);
      const char* in_row = in + (int64_t)b * a.in_sb;
      char* out_row = out + (int64_t)b * a.out_sb;
      for (int j0 = r0; j0 < npos; j0 += RSTEP * kUnroll) {
        V val[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int j = j0 + u * RSTEP;
          const int s = lo + j;
          val[u] = zero_vec<V>();
          if (j < npos) {
            if ((unsigned)(s - len) < (unsigned)T) {
              val[u] = ld_stream<V>(in_row + (int64_t)(s - len) * a.in_st + in_lane);
            } else if (s < hw) {
              const int blk = (int)a.div_page.div((uint32_t)s);
              const int64_t pb = __hip_readfirstlane(s_pbase[blk - blk_lo]);
              if (pb >= 0) val[u] = ld_stream<V>(pages + pb + (int64_t)(s - blk * P) * a.tok_bytes + page_lane);
            }
          }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int j = j0 + u * RSTEP;
          const int s = lo + j;
          if (j < npos) {
            if (a.gather) st_stream<V>(out_row + (int64_t)s * a.out_ss + out_lane, val[u]);
            if ((unsigned)(s - len) < (unsigned)T) {
              const int blk = (int)a.div_page.div((uint32_t)s);
              const int64_t pb = __hip_readfirstlane(s_pbase[blk - blk_lo]);
              if (pb >= 0) *(V*)(pages + pb + (int64_t)(s - blk * P) * a.tok_bytes + page_lane) = val[u];
            }
          }
        }
      }
    }
  } else if constexpr (LPP > 0) {
    // hv = 64 * LPP vectors per position, 32-bit offsets.  The four copy waves split a step of
    // RSTEP = 4 / LPP positions: wave w takes position (w - 1) / LPP of the step and column
    // block (w - 1) % LPP (vectors block * 64 + lane), so at every step the workgroup reads and
    // writes RSTEP whole adjacent rows; a wave's kUnroll loads cover positions r0, r0 + RSTEP, ...
    constexpr int RSTEP = 4 / LPP;
    constexpr int kSpan = RSTEP * kUnroll;  // positions one iteration of the workgroup covers
    if (wave > 0) {
      const int lane = (int)(threadIdx.x & (kWave - 1));
      const int r0 = __builtin_amdgcn_readfirstlane((wave - 1) / LPP);  // wave-uniform
      const int col = ((wave - 1) % LPP) * kWave + lane;
      const int h = (int)a.div_vr.div((uint32_t)col);
      const int v = col - h * (int)a.div_vr.d;
      const uint32_t page_lane = (uint32_t)(col * VB);
      const uint32_t out_lane = (uint32_t)((int64_t)h * a.out_sh + (int64_t)v * VB);
      const uint32_t in_lane = (uint32_t)((int64_t)h * a.in_sh + (int64_t)v * VB);
      const uint32_t tokb = (uint32_t)a.tok_bytes;
      const uint32_t oss = (uint32_t)a.out_ss;
      const uint32_t ist = (uint32_t)a.in_st;
      const char* in_row = in + (int64_t)b * a.in_sb;
      char* out_row = out + (int64_t)b * a.out_sb;
      const int ulen = __builtin_amdgcn_readfirstlane(len);
      const int uhw = __builtin_amdgcn_readfirstlane(hw);
      const int ulo = __builtin_amdgcn_readfirstlane(lo);
      const int unpos = __builtin_amdgcn_readfirstlane(npos);
      const int ublk_lo = __builtin_amdgcn_readfirstlane(blk_lo);
      for (int j0 = r0; j0 < unpos; j0 += kSpan) {
        const int nu = min(kUnroll, (unpos - j0 + RSTEP - 1) / RSTEP);  // positions in the tile
        const int sf = ulo + j0;                     // first position of this wave's iteration
        const int sl = sf + (nu - 1) * RSTEP;        // last
        const int bf = (int)a.div_page.div((uint32_t)sf);
        const int bl = (int)a.div_page.div((uint32_t)sl);
        const int64_t pb0 = __hip_readfirstlane(s_pbase[bf - ublk_lo]);
        const int64_t pb1 = __hip_readfirstlane(s_pbase[min(bf + 1 - ublk_lo, kMaxTilePages)]);
        const int64_t pb2 = __hip_readfirstlane(s_pbase[min(bf + 2 - ublk_lo, kMaxTilePages)]);
        if (bl <= bf + 2 && sl < max(uhw, ulen + T) && pb0 >= 0 && (bl < bf + 1 || pb1 >= 0) &&
            (bl < bf + 2 || pb2 >= 0)) {
          // Every position holds data (an earlier append, or a new token of this launch), on at
          // most three mapped pages.  Branch-free loads, back to back: positions past the tile
          // repeat the wave's last position (a cache hit) instead of branching, which would make
          // the compiler wait for each load.  Stores go one at a time (a single-round launch
          // drains HBM fastest with one store in flight per wave).
          const int split1 = (bf + 1) * P;           // first position of the second page
          const int split2 = split1 + P;             // and of the third
          V val[kUnroll];
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            const int s = sf + min(u, nu - 1) * RSTEP;
            const int64_t pb = s >= split2 ? pb2 : (s >= split1 ? pb1 : pb0);
            const int pstart = s >= split2 ? split2 : (s >= split1 ? split1 : split1 - P);
            const bool fresh = (unsigned)(s - ulen) < (unsigned)T;
            const char* base = fresh ? in_row + (uint32_t)(s - ulen) * ist : pages + pb + (uint32_t)(s - pstart) * tokb;
            val[u] = ld_stream<V>(base + (fresh ? in_lane : page_lane));
          }
          wait_vm<0>();
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) {
            if (u < nu) {
              const int s = sf + u * RSTEP;
              wait_vm<0>();
              if (a.gather) st_stream<V>((out_row + (uint32_t)s * oss) + out_lane, val[u]);
              if ((unsigned)(s - ulen) < (unsigned)T) {
                const int64_t pb = s >= split2 ? pb2 : (s >= split1 ? pb1 : pb0);
                const int pstart = s >= split2 ? split2 : (s >= split1 ? split1 : split1 - P);
                *(V*)((pages + pb + (uint32_t)(s - pstart) * tokb) + page_lane) = val[u];
              }
            }
          }
          continue;
        }
        V val[kUnroll];
        // Boundary iteration: the tile's last positions, new tokens, positions never written
        // (zero), stale positions past seq_lens, or more than two pages (small page sizes).
        // Taken in halves of kUnroll / 2 loads, which keeps the register footprint small.
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          constexpr int kHalf = kUnroll / 2;
#pragma unroll
          for (int k = 0; k < kHalf; ++k) {
            const int j = j0 + (half * kHalf + k) * RSTEP;
            const int s = ulo + j;
            val[k] = zero_vec<V>();
            if (j < unpos) {
              if ((unsigned)(s - ulen) < (unsigned)T) {
                val[k] = ld_stream<V>((in_row + (uint32_t)(s - ulen) * ist) + in_lane);
              } else if (s < uhw) {
                const int blk = (int)a.div_page.div((uint32_t)s);
                const int64_t pb = __hip_readfirstlane(s_pbase[blk - ublk_lo]);
                if (pb >= 0) val[k] = ld_stream<V>((pages + pb + (uint32_t)(s - blk * P) * tokb) + page_lane);
              }
            }
          }
#pragma unroll
          for (int k = 0; k < kHalf; ++k) {
            const int j = j0 + (half * kHalf + k) * RSTEP;
            const int s = ulo + j;
            if (j < unpos) {
              if (a.gather) st_stream<V>((out_row + (uint32_t)s * oss) + out_lane, val[k]);
              if ((unsigned)(s - ulen) < (unsigned)T) {
                const int blk = (int)a.div_page.div((uint32_t)s);
                const int64_t pb = __hip_readfirstlane(s_pbase[blk - ublk_lo]);
                if (pb >= 0) *(V*)((pages + pb + (uint32_t)(s - blk * P) * tokb) + page_lane) = val[k];
              }
            }
          }
        }
      }
    }
  } else {
    // Any geometry: copy thread i of the tile takes vectors i, i + kThreads, ... of the tile's
    // [positions, kv_heads * vr] run; only the data is held across the batch.
    const int total = npos * a.hv;
    const int64_t in_row = (int64_t)b * a.in_sb;
    const int64_t out_row = (int64_t)b * a.out_sb;
    for (int i0 = wave > 0 ? (int)threadIdx.x - kWave : total; i0 < total; i0 += kThreads * kUnroll) {
      V val[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = i0 + u * kThreads;
        val[u] = zero_vec<V>();
        if (i < total) {
          const int tok = (int)a.div_hv.div((uint32_t)i);
          const int hvi = i - tok * a.hv;
          const int s = lo + tok;
          if ((unsigned)(s - len) < (unsigned)T) {
            const int h = (int)a.div_vr.div((uint32_t)hvi);
            const int v = hvi - h * (int)a.div_vr.d;
            val[u] = ld_stream<V>(in + in_row + (int64_t)h * a.in_sh + (int64_t)(s - len) * a.in_st + (int64_t)v * VB);
          } else if (s < hw) {
            const int blk = (int)a.div_page.div((uint32_t)s);
            const int64_t pb = s_pbase[blk - blk_lo];
            if (pb >= 0) val[u] = ld_stream<V>(pages + pb + (int64_t)(s - blk * P) * a.tok_bytes + (int64_t)hvi * VB);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        const int i = i0 + u * kThreads;
        if (i < total) {
          const int tok = (int)a.div_hv.div((uint32_t)i);
          const int hvi = i - tok * a.hv;
          const int s = lo + tok;
          if (a.gather) {
            const int h = (int)a.div_vr.div((uint32_t)hvi);
            const int v = hvi - h * (int)a.div_vr.d;
            st_stream<V>(out + out_row + (int64_t)h * a.out_sh + (int64_t)s * a.out_ss + (int64_t)v * VB, val[u]);
          }
          if ((unsigned)(s - len) < (unsigned)T) {
            const int blk = (int)a.div_page.div((uint32_t)s);
            const int64_t pb = s_pbase[blk - blk_lo];
            if (pb >= 0) *(V*)(pages + pb + (int64_t)(s - blk * P) * a.tok_bytes + (int64_t)hvi * VB) = val[u];
          }
        }
      }
    }
  }

  if (committing && !early) {
    // More rows than a wave has lanes: arrive after the copy; the last tile commits with the
    // whole workgroup.
    __syncthreads();
    if (threadIdx.x == 0) s_meta[5] = atomicAdd(&p.ctrl[BARQ_KV_CTRL_ARRIVED], 1) == (int)gridDim.x - 1;
    __syncthreads();
    if (s_meta[5]) {
      commit_append<kStreamThreads>(p, a.batch, T, a.gather ? a.seq_out : INT_MAX, a.div_page);
      if (threadIdx.x == 0) atomicExch(&p.ctrl[BARQ_KV_CTRL_ARRIVED], 0);
    }
  }
}

// The unit-mapped kernels hold 16 vectors per copy thread; five waves per SIMD keep four tiles
// resident per CU (their few spills sit on the new-token path).  The generic kernel keeps the
// compiler's register allocation.
template <int VB, int LPP>
__global__ void __launch_bounds__(kStreamThreads) __attribute__((amdgpu_waves_per_eu(5)))
stream_kernel(const StreamArgs a) {
  stream_body<VB, LPP, false>(a);
}

template <int VB, int LPP>
__global__ void __launch_bounds__(kStreamThreads) stream_kernel_rounds(const StreamArgs a) {
  stream_body<VB, LPP, true>(a);
}

template <int VB>
__global__ void __launch_bounds__(kStreamThreads) stream_kernel_any(const StreamArgs a) {
  stream_body<VB, 0, false>(a);
}

// ---------------------------------------------------------------------------------------------
// Lean gather / update: launches whose tiles of one or two pages are all resident at once
// (batch <= 64, whole-row geometry, 16-byte vectors).  Every copy wave reads its own tile's
// metadata -- the row's length and mark, the block-table entries of the tile's blocks -- with
// uniform loads, served by the scalar cache, and starts streaming without LDS staging; batch-wide
// values (the longest row, the rank of a row's new blocks) are read only by the tiles that need
// them.  Wave 0 only counts the tile as arrived, after a barrier that follows every copy wave's
// metadata loads, and in the last tile to arrive commits the append.  Measured at the C2 shape
// against the control-wave kernel above (gather at context 520..760): 1-page tiles 13.2-14.9 us
// against 14.8-16.3 us while at most five tiles per CU exist, 2-page tiles 14.6-17.0 us against
// 16.0-18.0 us beyond.
// ---------------------------------------------------------------------------------------------

// Lean tiles resident on one CU: five at up to 8 vectors per copy thread (<= 64 VGPRs), four at
// 16 (75 VGPRs: six waves per SIMD).
constexpr int64_t kLeanResidentTilesPerCU = 5;
constexpr int64_t kLeanResidentTilesPerCU16 = 4;
// Known-state launches of at most this many tiles store back to back (batch 1 at the C2 shape,
// context 650: 5.08 -> 4.97 us per launch); larger ones keep one store in flight per wave.
constexpr unsigned kKnownBackToBackTiles = 256;

// Page of block `blk`, the k-th block a lean tile touches (touched = nbl - k > 0): its table
// entry for an old block, the stack entry of its rank for a new one; -1 when unmapped.
__device__ __forceinline__ int lean_page(const barq_kv_pool& p, const NewBlocks& nb, int blk, int touched, int mb,
                                         int top, int base, int entry) {
  if (touched <= 0 || blk >= mb) return -1;
  if (blk < nb.first) return checked_page(entry, p.num_pages);
  if (blk < nb.first + nb.count) {
    const int idx = top - 1 - (base + blk - nb.first);
    return idx >= 0 ? checked_page(p.free_pages[idx], p.num_pages) : -1;
  }
  return -1;
}

// NU: vectors per copy thread (positions per tile / (4 / LPP)); tiles are whole pages, at most two.
// (lean_balanced_kernel below takes launches whose one-page tiles are cut into equal chunks.)
template <int NU, int LPP>
__global__ void __launch_bounds__(kStreamThreads) lean_stream_kernel(const StreamArgs a) {
  using V = typename VecT<16>::T;
  constexpr int RSTEP = 4 / LPP;
  const barq_kv_pool& p = a.pool;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int bid = (int)blockIdx.x;
  const int kv = bid & 1;
  const int rest = bid >> 1;
  const int b = (int)a.div_chunks.div((uint32_t)rest);
  const int c = rest - b * (int)a.div_chunks.d;
  const int T = a.tokens;
  const int P = (int)p.page_size;
  const int mb = (int)p.max_blocks;
  const bool committing = T > 0 && a.commit_in_kernel;
  __shared__ int s_ready;  // copy waves whose metadata loads have returned (committing tiles)
  if (committing) {
    if (wave == 0 && lane == 0) s_ready = 0;
    __syncthreads();
  }

  if (wave == 0) {
    if (!committing) return;
    // The tile arrives once every copy wave holds the metadata it uses: the copy waves count
    // themselves in LDS instead of waiting for each other at a barrier.
    while (__hip_atomic_load(&s_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < kCopyWaves)
      __builtin_amdgcn_s_sleep(1);
    arrive_and_commit(p, a.nsub, a.batch, T, a.seq_out, a.div_page);
    return;
  }

  // Copy waves.  Tile (K or V, row b, chunk c): positions [c * chunk, + chunk), blocks blk0 and,
  // for two-page tiles, blk0 + 1 (< max_blocks: the grid covers seq_out <= capacity).
  const int len = p.seq_lens[b];
  const int hw = p.high_water[b];
  const int blk0 = c * a.ppt;
  const int64_t trow = (int64_t)b * mb;
  const int e0 = p.block_table[trow + blk0];
  const int e1_read = p.block_table[trow + min(blk0 + 1, mb - 1)];
  // The arguments the copies address with are requested in the metadata's round trip (left to
  // itself the compiler asks for them only once the metadata has arrived: one more round trip
  // before the first page load).  Loads after this point are vector loads.
  asm volatile("" ::"s"(a.in_k), "s"(a.in_v), "s"(a.out_k), "s"(a.out_v), "s"(a.in_sb), "s"(a.in_sh), "s"(a.in_st),
               "s"(a.out_sb), "s"(a.out_sh), "s"(a.out_ss), "s"(a.page_bytes), "s"(a.tok_bytes));
  const int e1 = (a.ppt > 1 && blk0 + 1 < mb) ? e1_read : -1;
  const int lo = c * a.chunk;
  int hi = lo + a.chunk;
  if (hi > min(len + T, a.seq_out)) {
    // Positions past this row's end: the output extent is the longest row (or seq_out).
    int smax = a.seq_out;
    if (a.seq_from_device) smax = min(wave_max(lane < a.batch ? p.seq_lens[lane] + T : 0), a.seq_out);
    hi = min(hi, smax);
  }
  const NewBlocks nb = new_blocks(len, hw, T, mb, a.div_page);
  const int nbl = a.ppt > 1 ? 2 : 1;
  int base = 0, top = 0;
  if (nb.count > 0 && blk0 < nb.first + nb.count && blk0 + nbl > nb.first) {
    // The tile holds new blocks: their pages are ranked after the new blocks of rows [0, b).
    top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
    base = wave_sum(lane < b ? new_blocks(p.seq_lens[lane], p.high_water[lane], T, mb, a.div_page).count : 0);
  }
  int64_t pbs[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int blk = blk0 + k;
    int page = -1;
    if (k < nbl && blk < mb) {
      if (blk < nb.first) {
        page = checked_page(k == 0 ? e0 : e1, p.num_pages);
      } else if (blk < nb.first + nb.count) {
        const int idx = top - 1 - (base + blk - nb.first);
        page = idx >= 0 ? checked_page(p.free_pages[idx], p.num_pages) : -1;
      }
    }
    pbs[k] = page >= 0 ? (int64_t)page * a.page_bytes : (int64_t)-1;
  }
  const int64_t pb0 = pbs[0], pb1 = pbs[1];
  if (committing) {
    // Counted once the values have returned: the asm consumes every metadata value the tile read
    // (the compiler waits for them before it), and the count follows it.
    asm volatile("" ::"s"(len), "s"(hw), "s"(e0), "s"(e1), "s"(top), "s"(base), "s"(hi), "s"(pb0), "s"(pb1));
    if (lane == 0) __hip_atomic_fetch_add(&s_ready, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (hi <= lo) return;

  const int cw = wave - 1;
  const int r0 = cw / LPP;
  const int col = (cw % LPP) * kWave + lane;
  const int h = (int)a.div_vr.div((uint32_t)col);
  const int v = col - h * (int)a.div_vr.d;
  const uint32_t page_lane = (uint32_t)(col * 16);
  const uint32_t out_lane = (uint32_t)((int64_t)h * a.out_sh + (int64_t)v * 16);
  const uint32_t in_lane = (uint32_t)((int64_t)h * a.in_sh + (int64_t)v * 16);
  const uint32_t tokb = (uint32_t)a.tok_bytes;
  const uint32_t oss = (uint32_t)a.out_ss;
  const uint32_t ist = (uint32_t)a.in_st;
  const char* in_row = (kv ? a.in_v : a.in_k) + (int64_t)b * a.in_sb;
  char* out_row = (kv ? a.out_v : a.out_k) + (int64_t)b * a.out_sb;
  char* pages = (char*)(kv ? p.value_pages : p.key_pages);
  const int nval = hi - lo;
  V val[NU];
  if (hi <= max(hw, len + T) && pb0 >= 0 && (nval <= P || pb1 >= 0)) {
    // Every position holds data on mapped pages: branch-free loads, back to back (positions past
    // the tile repeat its last one, a cache hit).
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int j = min(r0 + u * RSTEP, nval - 1);
      const int s = lo + j;
      const bool second = j >= P;
      const char* page_pos = pages + (second ? pb1 : pb0) + (uint32_t)(second ? j - P : j) * tokb;
      const bool fresh = (unsigned)(s - len) < (unsigned)T;
      val[u] = ld_stream<V>(fresh ? in_row + (uint32_t)(s - len) * ist + in_lane : page_pos + page_lane);
    }
  } else {
    // Zero padding, unmapped blocks (an exhausted pool) or positions never written.
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int j = r0 + u * RSTEP;
      const int s = lo + j;
      val[u] = zero_vec<V>();
      if (j < nval) {
        const bool second = j >= P;
        const int64_t pb = second ? pb1 : pb0;
        if ((unsigned)(s - len) < (unsigned)T) {
          val[u] = ld_stream<V>(in_row + (uint32_t)(s - len) * ist + in_lane);
        } else if (s < hw && pb >= 0) {
          val[u] = ld_stream<V>(pages + pb + (uint32_t)(second ? j - P : j) * tokb + page_lane);
        }
      }
    }
  }
  wait_vm<0>();
  // One store in flight per wave: a single-round launch drains HBM fastest that way.
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int j = r0 + u * RSTEP;
    if (j < nval) {
      const int s = lo + j;
      wait_vm<0>();
      st_stream<V>(out_row + (uint32_t)s * oss + out_lane, val[u]);
      if ((unsigned)(s - len) < (unsigned)T) {
        const bool second = j >= P;
        const int64_t pb = second ? pb1 : pb0;
        if (pb >= 0) *(V*)(pages + pb + (uint32_t)(second ? j - P : j) * tokb + page_lane) = val[u];
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Lean update with the row state known to the caller (barq_kv_update_known: an eager caller whose
// host shadow holds the rows' lengths and marks and the stack top exactly).  The state arrives
// in the kernel arguments, so no tile reads seq_lens, high_water or the stack top, and the
// commit cannot race a tile's read: the first tile's control wave commits at once, with no
// arrival counters.  The block-table entries a tile reads (blocks mapped before the launch) and
// the stack entries new blocks take are not written by the commit.  A launch of at most one
// tile per CU (the memory system far from busy) issues its stores back to back.
// ---------------------------------------------------------------------------------------------

struct KnownState {
  int32_t len[kWave];
  int32_t hw[kWave];
  int32_t top;
};

template <int NU, int LPP>
__global__ void __launch_bounds__(kStreamThreads) lean_known_kernel(const StreamArgs a, const KnownState ks) {
  using V = typename VecT<16>::T;
  constexpr int RSTEP = 4 / LPP;
  const barq_kv_pool& p = a.pool;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int bid = (int)blockIdx.x;
  const int T = a.tokens;
  const int mb = (int)p.max_blocks;

  if (wave == 0) {
    if (bid != 0 || T <= 0) return;
    const int clen = lane < a.batch ? ks.len[lane] : 0;
    const int chw = lane < a.batch ? ks.hw[lane] : 0;
    const int news = wave_sum(lane < a.batch ? new_blocks(clen, chw, T, mb, a.div_page).count : 0);
    const int fidx = ks.top - 1 - lane;
    const int cfree = news > 0 && fidx >= 0 ? p.free_pages[fidx] : -1;
    commit_from_lanes(p, a.batch, T, a.seq_out, a.div_page, clen, chw, ks.top, cfree);
    return;
  }

  const int kv = bid & 1;
  const int rest = bid >> 1;
  const int b = (int)a.div_chunks.div((uint32_t)rest);
  const int c = rest - b * (int)a.div_chunks.d;
  const int P = (int)p.page_size;
  const int len = ks.len[b];
  const int hw = ks.hw[b];
  const int blk0 = c * a.ppt;
  const int e0 = p.block_table[(int64_t)b * mb + blk0];
  int e1 = -1;
  if (a.ppt > 1 && blk0 + 1 < mb) e1 = p.block_table[(int64_t)b * mb + blk0 + 1];
  const int lo = c * a.chunk;
  const int hi = min(lo + a.chunk, a.seq_out);
  if (hi <= lo) return;
  const NewBlocks nb = new_blocks(len, hw, T, mb, a.div_page);
  const int nbl = a.ppt > 1 ? 2 : 1;
  int base = 0;
  if (nb.count > 0 && blk0 < nb.first + nb.count && blk0 + nbl > nb.first)
    base = wave_sum(lane < b ? new_blocks(ks.len[lane], ks.hw[lane], T, mb, a.div_page).count : 0);
  const int pg0 = lean_page(p, nb, blk0, nbl, mb, ks.top, base, e0);
  const int pg1 = lean_page(p, nb, blk0 + 1, nbl - 1, mb, ks.top, base, e1);
  const int64_t pb0 = pg0 >= 0 ? (int64_t)pg0 * a.page_bytes : (int64_t)-1;
  const int64_t pb1 = pg1 >= 0 ? (int64_t)pg1 * a.page_bytes : (int64_t)-1;

  const int cw = wave - 1;
  const int r0 = cw / LPP;
  const int col = (cw % LPP) * kWave + lane;
  const int h = (int)a.div_vr.div((uint32_t)col);
  const int v = col - h * (int)a.div_vr.d;
  const uint32_t page_lane = (uint32_t)(col * 16);
  const uint32_t out_lane = (uint32_t)((int64_t)h * a.out_sh + (int64_t)v * 16);
  const uint32_t in_lane = (uint32_t)((int64_t)h * a.in_sh + (int64_t)v * 16);
  const uint32_t tokb = (uint32_t)a.tok_bytes;
  const uint32_t oss = (uint32_t)a.out_ss;
  const uint32_t ist = (uint32_t)a.in_st;
  const char* in_row = (kv ? a.in_v : a.in_k) + (int64_t)b * a.in_sb;
  char* out_row = (kv ? a.out_v : a.out_k) + (int64_t)b * a.out_sb;
  char* pages = (char*)(kv ? p.value_pages : p.key_pages);
  const int nval = hi - lo;
  V val[NU];
  if (hi <= max(hw, len + T) && pb0 >= 0 && (nval <= P || pb1 >= 0)) {
    // Every position holds data on mapped pages: branch-free loads, back to back (positions past
    // the tile repeat its last one, a cache hit).
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int j = min(r0 + u * RSTEP, nval - 1);
      const int s = lo + j;
      const bool second = j >= P;
      const char* page_pos = pages + (second ? pb1 : pb0) + (uint32_t)(second ? j - P : j) * tokb;
      const bool fresh = (unsigned)(s - len) < (unsigned)T;
      val[u] = ld_stream<V>(fresh ? in_row + (uint32_t)(s - len) * ist + in_lane : page_pos + page_lane);
    }
  } else {
    // Zero padding, unmapped blocks (an exhausted pool) or positions never written.
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int j = r0 + u * RSTEP;
      const int s = lo + j;
      val[u] = zero_vec<V>();
      if (j < nval) {
        const bool second = j >= P;
        const int64_t pb = second ? pb1 : pb0;
        if ((unsigned)(s - len) < (unsigned)T) {
          val[u] = ld_stream<V>(in_row + (uint32_t)(s - len) * ist + in_lane);
        } else if (s < hw && pb >= 0) {
          val[u] = ld_stream<V>(pages + pb + (uint32_t)(second ? j - P : j) * tokb + page_lane);
        }
      }
    }
  }
  const bool paced = gridDim.x > kKnownBackToBackTiles;
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int j = r0 + u * RSTEP;
    if (j < nval) {
      const int s = lo + j;
      if (paced) wait_vm<0>();
      st_stream<V>(out_row + (uint32_t)s * oss + out_lane, val[u]);
      if ((unsigned)(s - len) < (unsigned)T) {
        const bool second = j >= P;
        const int64_t pb = second ? pb1 : pb0;
        if (pb >= 0) *(V*)(pages + pb + (uint32_t)(second ? j - P : j) * tokb + page_lane) = val[u];
      }
    }
  }
}

// Balanced lean tiles: lean_stream_kernel's work for chunks that start anywhere in a page.
// NU: vectors per copy thread; a chunk holds at most one page of positions (NU * 4 / LPP).
template <int NU, int LPP>
__global__ void __launch_bounds__(kStreamThreads) lean_balanced_kernel(const StreamArgs a) {
  using V = typename VecT<16>::T;
  constexpr int RSTEP = 4 / LPP;
  const barq_kv_pool& p = a.pool;
  const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  const int lane = (int)(threadIdx.x & (kWave - 1));
  const int bid = (int)blockIdx.x;
  const int kv = bid & 1;
  const int rest = bid >> 1;
  const int b = (int)a.div_chunks.div((uint32_t)rest);
  const int c = rest - b * (int)a.div_chunks.d;
  const int T = a.tokens;
  const int P = (int)p.page_size;
  const int mb = (int)p.max_blocks;
  const bool committing = T > 0 && a.commit_in_kernel;

  // (The LDS count of lean_stream_kernel, in place of this barrier, cost the balanced tiles
  // ~1 %: their copy waves get their metadata late, and the control waves poll meanwhile.)
  if (wave == 0) {
    if (!committing) return;
    __syncthreads();  // every copy wave of the tile holds the metadata it uses
    arrive_and_commit(p, a.nsub, a.batch, T, a.seq_out, a.div_page);
    return;
  }

  // Copy waves.  Tile (K or V, row b, chunk c): the row's positions up to its new end, [0, L) with
  // L = min(len + T, seq_out), cut into m = div_chunks.d equal chunks (ceil(L / m) positions,
  // at most a tile's NU * 4 / LPP), so that every tile of the launch -- and every CU, the grid
  // being a multiple of the CU count -- moves the same bytes whatever the context.  The output
  // positions past the row's end, [L, E) up to the extent E (stale data below the mark, else
  // zeros), are cut the same way when E = seq_out is known here, else (extent on the device)
  // written by the row's last chunk.  Balanced tiles hold at most one page of positions, so a
  // chunk at page offset `off` touches at most two blocks, as a two-page tile does.
  const int len = p.seq_lens[b];
  const int hw = p.high_water[b];
  const int64_t trow = (int64_t)b * mb;
  int lo, hi, xlo = 0, xhi = 0, blk0, off = 0, nbl, e0 = -1, e1 = -1;
  {
    const int m = (int)a.div_chunks.d;
    const int L = min(len + T, a.seq_out);
    const int q = (int)a.div_chunks.div((uint32_t)(L + m - 1));
    lo = min(c * q, L);
    hi = min(lo + q, L);
    if (!a.seq_from_device) {
      const int z = (int)a.div_chunks.div((uint32_t)(a.seq_out - L + m - 1));
      xlo = min(L + c * z, a.seq_out);
      xhi = min(xlo + z, a.seq_out);
    } else if (c == m - 1) {
      xlo = L;
      xhi = min(wave_max(lane < a.batch ? p.seq_lens[lane] + T : 0), a.seq_out);
    }
    blk0 = (int)a.div_page.div((uint32_t)lo);
    off = lo - blk0 * P;
    nbl = hi > lo ? (int)a.div_page.div((uint32_t)(off + hi - lo - 1)) + 1 : 0;  // blocks touched
    if (nbl > 0) e0 = p.block_table[trow + blk0];
    if (nbl > 1 && blk0 + 1 < mb) e1 = p.block_table[trow + blk0 + 1];
  }

  const NewBlocks nb = new_blocks(len, hw, T, mb, a.div_page);
  int base = 0, top = 0;
  if (nb.count > 0 && blk0 < nb.first + nb.count && blk0 + nbl > nb.first) {
    // The tile holds new blocks: their pages are ranked after the new blocks of rows [0, b).
    top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
    base = wave_sum(lane < b ? new_blocks(p.seq_lens[lane], p.high_water[lane], T, mb, a.div_page).count : 0);
  }
  const int pg0 = lean_page(p, nb, blk0, nbl, mb, top, base, e0);
  const int pg1 = lean_page(p, nb, blk0 + 1, nbl - 1, mb, top, base, e1);
  const int64_t pb0 = pg0 >= 0 ? (int64_t)pg0 * a.page_bytes : (int64_t)-1;
  const int64_t pb1 = pg1 >= 0 ? (int64_t)pg1 * a.page_bytes : (int64_t)-1;
  if (committing) {
    __builtin_amdgcn_s_waitcnt(0);  // the metadata loads have returned before the tile arrives
    __syncthreads();
  }
  if (hi <= lo && xhi <= xlo) return;

  const int cw = wave - 1;
  const int r0 = cw / LPP;
  const int col = (cw % LPP) * kWave + lane;
  const int h = (int)a.div_vr.div((uint32_t)col);
  const int v = col - h * (int)a.div_vr.d;
  const uint32_t page_lane = (uint32_t)(col * 16);
  const uint32_t out_lane = (uint32_t)((int64_t)h * a.out_sh + (int64_t)v * 16);
  const uint32_t in_lane = (uint32_t)((int64_t)h * a.in_sh + (int64_t)v * 16);
  const uint32_t tokb = (uint32_t)a.tok_bytes;
  const uint32_t oss = (uint32_t)a.out_ss;
  const uint32_t ist = (uint32_t)a.in_st;
  const char* in_row = (kv ? a.in_v : a.in_k) + (int64_t)b * a.in_sb;
  char* out_row = (kv ? a.out_v : a.out_k) + (int64_t)b * a.out_sb;
  char* pages = (char*)(kv ? p.value_pages : p.key_pages);
  const int nval = hi - lo;
  V val[NU];
  if (nval > 0) {
    if (hi <= max(hw, len + T) && pb0 >= 0 && (nbl < 2 || pb1 >= 0)) {
      // Every position holds data on mapped pages: branch-free loads, back to back (positions
      // past the tile repeat its last one, a cache hit).
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int j = min(r0 + u * RSTEP, nval - 1);
        const int s = lo + j;
        const bool fresh = (unsigned)(s - len) < (unsigned)T;
        const int w = off + j;
        const bool second = w >= P;
        const char* page_at = pages + (second ? pb1 : pb0) + (uint32_t)(second ? w - P : w) * tokb;
        val[u] = ld_stream<V>(fresh ? in_row + (uint32_t)(s - len) * ist + in_lane : page_at + page_lane);
      }
    } else {
      // Zero padding, unmapped blocks (an exhausted pool) or positions never written.
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const int j = r0 + u * RSTEP;
        const int s = lo + j;
        val[u] = zero_vec<V>();
        if (j < nval) {
          const int w = off + j;
          const bool second = w >= P;
          const int64_t pb = second ? pb1 : pb0;
          if ((unsigned)(s - len) < (unsigned)T) {
            val[u] = ld_stream<V>(in_row + (uint32_t)(s - len) * ist + in_lane);
          } else if (s < hw && pb >= 0) {
            val[u] = ld_stream<V>(pages + pb + (uint32_t)(second ? w - P : w) * tokb + page_lane);
          }
        }
      }
    }
    wait_vm<0>();
    // One store in flight per wave: a single-round launch drains HBM fastest that way.
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int j = r0 + u * RSTEP;
      if (j < nval) {
        const int s = lo + j;
        wait_vm<0>();
        st_stream<V>(out_row + (uint32_t)s * oss + out_lane, val[u]);
        if ((unsigned)(s - len) < (unsigned)T) {
          const int w = off + j;
          const bool second = w >= P;
          const int64_t pb = second ? pb1 : pb0;
          if (pb >= 0) *(V*)(pages + pb + (uint32_t)(second ? w - P : w) * tokb + page_lane) = val[u];
        }
      }
    }
  }
  // Balanced tiles: output positions [xlo, xhi) past the row's new end (no new tokens there):
  // stale data below the mark on the pages the table maps (blocks below the mark are old ones,
  // which the commit does not remap), else zeros.
  for (int s0 = xlo; s0 < xhi; s0 += NU * RSTEP) {
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int s = s0 + r0 + u * RSTEP;
      val[u] = zero_vec<V>();
      if (s < xhi && s < hw) {
        const int blk = (int)a.div_page.div((uint32_t)s);
        const int page = checked_page(p.block_table[trow + blk], p.num_pages);
        if (page >= 0)
          val[u] = ld_stream<V>(pages + (int64_t)page * a.page_bytes + (uint32_t)(s - blk * P) * tokb + page_lane);
      }
    }
    wait_vm<0>();
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int s = s0 + r0 + u * RSTEP;
      if (s < xhi) {
        wait_vm<0>();
        st_stream<V>(out_row + (uint32_t)s * oss + out_lane, val[u]);
      }
    }
  }
}

__global__ void __launch_bounds__(kThreads) commit_kernel(const barq_kv_pool p, int batch,
                                                         int tokens, int limit, FastDiv div_page) {
  commit_append<kThreads>(p, batch, tokens, limit, div_page);
}

// ---------------------------------------------------------------------------------------------
// Dense drop-in (reference layout [cache_batch, H, max_blocks, P, D]).
// ---------------------------------------------------------------------------------------------

struct DenseArgs {
  char* kc;
  char* vc;
  const int32_t* seq_lens;
  const char* ks;
  const char* vs;
  int64_t sb, sh, st;  // bytes
  int64_t row_bytes;
  int32_t heads, tokens, max_blocks, page_size;
  int32_t total;       // batch * heads * tokens * vr
  FastDiv div_vr, div_tokens, div_heads, div_page;
};

template <int VB>
__global__ void __launch_bounds__(kThreads) dense_append_kernel(const DenseArgs a) {
  using V = typename VecT<VB>::T;
  const int stride = (int)(gridDim.x * kThreads);
  for (int i0 = blockIdx.x * kThreads + threadIdx.x; i0 < a.total; i0 += stride * kUnroll) {
    V kval[kUnroll], vval[kUnroll];
    int64_t dst[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = i0 + u * stride;
      dst[u] = -1;
      kval[u] = zero_vec<V>();
      vval[u] = zero_vec<V>();
      if (i < a.total) {
        // i -> (b, h, t, v) over [batch, heads, tokens, vectors per row]
        const int row = (int)a.div_vr.div((uint32_t)i);
        const int v = i - row * (int)a.div_vr.d;
        const int bh = (int)a.div_tokens.div((uint32_t)row);
        const int t = row - bh * a.tokens;
        const int b = (int)a.div_heads.div((uint32_t)bh);
        const int h = bh - b * a.heads;
        const int pos = a.seq_lens[b] + t;
        const int blk = (int)a.div_page.div((uint32_t)pos);
        if (blk < a.max_blocks) {  // paged_kv_cache.cu:42-44 skips slots past the last block
          const int off = pos - blk * a.page_size;
          const int64_t src = (int64_t)b * a.sb + (int64_t)h * a.sh + (int64_t)t * a.st + (int64_t)v * VB;
          dst[u] = (((int64_t)bh * a.max_blocks + blk) * a.page_size + off) * a.row_bytes + (int64_t)v * VB;
          kval[u] = *(const V*)(a.ks + src);
          vval[u] = *(const V*)(a.vs + src);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      if (dst[u] >= 0) {
        *(V*)(a.kc + dst[u]) = kval[u];
        *(V*)(a.vc + dst[u]) = vval[u];
      }
    }
  }
}

__global__ void dense_bump_kernel(int32_t* seq_lens, int batch, int tokens) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < batch) seq_lens[i] += tokens;
}

// ---------------------------------------------------------------------------------------------
// Pool bookkeeping.
// ---------------------------------------------------------------------------------------------

__global__ void reset_kernel(const barq_kv_pool p, const int32_t* order) {
  const int64_t n_pages = p.num_pages;
  const int64_t n_table = p.max_batch * p.max_blocks;
  int64_t n = n_pages > n_table ? n_pages : n_table;
  if (n < p.max_batch) n = p.max_batch;
  if (n < BARQ_KV_CTRL_WORDS) n = BARQ_KV_CTRL_WORDS;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    // Stack entry i is popped (num_pages - 1 - i)-th, so page_order[k] is the k-th page taken.
    if (i < n_pages) p.free_pages[i] = order ? order[n_pages - 1 - i] : (int32_t)(n_pages - 1 - i);
    if (i < n_pages && p.page_shares) p.page_shares[i] = 0;
    if (i < n_table) p.block_table[i] = -1;
    if (i < p.max_batch) {
      p.seq_lens[i] = 0;
      p.high_water[i] = 0;
    }
    if (i < BARQ_KV_CTRL_WORDS) p.ctrl[i] = (i == BARQ_KV_CTRL_FREE_TOP) ? (int32_t)n_pages : 0;
  }
}

__global__ void crop_kernel(int32_t* seq_lens, int batch, int max_length) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < batch) seq_lens[i] = min(seq_lens[i], max_length);
}

// One workgroup: drop the listed rows' references, a row at a time with its blocks spread over
// the threads.  A page that no block holds any more is pushed back on the stack, in (row, block)
// order; with page_shares, a shared page only loses a reference.
__global__ void __launch_bounds__(kThreads) free_rows_kernel(const barq_kv_pool p,
                                                            const int32_t* rows, int n,
                                                            FastDiv div_page) {
  __shared__ int lds_scan[kWaves];
  const int top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
  const int mb = (int)p.max_blocks;
  int pushed = 0;
  int err = 0;
  for (int i = 0; i < n; ++i) {
    const int r = rows[i];
    if (r < 0 || r >= (int)p.max_batch) {
      err |= BARQ_KV_ERRBIT_BAD_INDEX;
      continue;
    }
    const int cnt = min(ceil_div_fd(p.high_water[r], div_page), mb);
    int32_t* row = p.block_table + (int64_t)r * mb;
    constexpr int kGroup = 4;  // chunks of kThreads blocks whose entries are read together
    for (int g0 = 0; g0 < cnt; g0 += kGroup * kThreads) {
      int entry[kGroup];
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const int j = g0 + u * kThreads + (int)threadIdx.x;
        entry[u] = j < cnt ? row[j] : -1;
      }
#pragma unroll
      for (int u = 0; u < kGroup; ++u) {
        const int j0 = g0 + u * kThreads;
        if (j0 >= cnt) break;
        const int j = j0 + (int)threadIdx.x;
        int page = -1, freed = 0;
        if (j < cnt) {
          page = checked_page(entry[u], p.num_pages);
          freed = page >= 0;
          if (freed && p.page_shares) {
            freed = atomicSub(&p.page_shares[page], 1) == 0;
            if (freed) p.page_shares[page] = 0;
          }
          row[j] = -1;
        }
        int chunk_total = 0;
        const int excl = block_exclusive_scan<kWaves>(freed, lds_scan, &chunk_total);
        if (freed) {
          const int64_t slot = (int64_t)top + pushed + excl;
          if (slot < p.num_pages) p.free_pages[slot] = page;
          else err |= BARQ_KV_ERRBIT_BAD_INDEX;
        }
        pushed += chunk_total;
      }
    }
    __syncthreads();  // every thread has read the row's mark before it is cleared
    if (threadIdx.x == 0) {
      p.seq_lens[r] = 0;
      p.high_water[r] = 0;
    }
  }
  if (threadIdx.x == 0) p.ctrl[BARQ_KV_CTRL_FREE_TOP] = (int)min((int64_t)top + pushed, p.num_pages);
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// Workgroup-wide copy of nvec vectors of VB bytes.
template <int VB>
__device__ __forceinline__ void copy_run(const char* src, char* dst, int nvec) {
  using V = typename VecT<VB>::T;
  for (int v0 = threadIdx.x; v0 < nvec; v0 += kThreads * kUnroll) {
    V val[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int v = v0 + u * kThreads;
      val[u] = v < nvec ? *(const V*)(src + (int64_t)v * VB) : zero_vec<V>();
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int v = v0 + u * kThreads;
      if (v < nvec) *(V*)(dst + (int64_t)v * VB) = val[u];
    }
  }
}

// Copy rows: tile = (dst row i, block j) copies one K page and one V page.
struct CopyArgs {
  barq_kv_pool src;
  barq_kv_pool dst;
  const int32_t* rows;
  int32_t n;
  int64_t page_bytes;
  FastDiv div_page;
  FastDiv div_blocks;
};

template <int VB>
__global__ void __launch_bounds__(kThreads) copy_rows_kernel(const CopyArgs a) {
  using V = typename VecT<VB>::T;
  __shared__ int s_meta[3];  // src page, dst page, last
  const int mb = (int)a.src.max_blocks;
  const int i = (int)a.div_blocks.div(blockIdx.x);
  const int j = (int)blockIdx.x - i * mb;

  if (threadIdx.x < kWave) {
    const int lane = threadIdx.x;
    // Rank base: blocks of dst rows [0, i).
    int acc = 0;
    for (int q0 = 0; q0 < i; q0 += kWave) {
      const int q = q0 + lane;
      int c = 0;
      if (q < i) {
        const int r = a.rows[q];
        if (r >= 0 && r < (int)a.src.max_batch) c = min(ceil_div_fd(a.src.high_water[r], a.div_page), mb);
      }
      acc += wave_sum(c);
    }
    if (lane == 0) {
      const int r = a.rows[i];
      int sp = -1, dp = -1;
      if (r >= 0 && r < (int)a.src.max_batch && j < min(ceil_div_fd(a.src.high_water[r], a.div_page), mb)) {
        sp = checked_page(a.src.block_table[(int64_t)r * mb + j], a.src.num_pages);
        const int idx = a.dst.ctrl[BARQ_KV_CTRL_FREE_TOP] - 1 - (acc + j);
        dp = idx >= 0 ? checked_page(a.dst.free_pages[idx], a.dst.num_pages) : -1;
      }
      s_meta[0] = sp;
      s_meta[1] = dp;
    }
  }
  __syncthreads();
  const int sp = s_meta[0];
  const int dp = s_meta[1];
  if (sp >= 0 && dp >= 0) {
    const int nvec = (int)(a.page_bytes / VB);
    copy_run<VB>((const char*)a.src.key_pages + (int64_t)sp * a.page_bytes,
                 (char*)a.dst.key_pages + (int64_t)dp * a.page_bytes, nvec);
    copy_run<VB>((const char*)a.src.value_pages + (int64_t)sp * a.page_bytes,
                 (char*)a.dst.value_pages + (int64_t)dp * a.page_bytes, nvec);
  }

  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(&a.dst.ctrl[BARQ_KV_CTRL_ARRIVED], 1);
    s_meta[2] = (prev == (int)gridDim.x - 1);
  }
  __syncthreads();
  if (!s_meta[2]) return;

  // Last tile: commit dst metadata.
  __shared__ int lds_scan[kWaves];
  const int top = a.dst.ctrl[BARQ_KV_CTRL_FREE_TOP];
  int used = 0, err = 0;
  for (int q0 = 0; q0 < a.n; q0 += kThreads) {
    const int q = q0 + (int)threadIdx.x;
    int r = -1, cnt = 0;
    if (q < a.n) {
      r = a.rows[q];
      if (r < 0 || r >= (int)a.src.max_batch) {
        err |= BARQ_KV_ERRBIT_BAD_INDEX;
        r = -1;
      } else {
        cnt = min(ceil_div_fd(a.src.high_water[r], a.div_page), mb);
      }
    }
    int chunk_total = 0;
    const int excl = block_exclusive_scan<kWaves>(cnt, lds_scan, &chunk_total);
    if (q < a.n) {
      for (int jj = 0; jj < cnt; ++jj) {
        const int idx = top - 1 - (used + excl + jj);
        const int page = idx >= 0 ? checked_page(a.dst.free_pages[idx], a.dst.num_pages) : -1;
        if (page < 0) err |= BARQ_KV_ERRBIT_POOL_EXHAUSTED;
        a.dst.block_table[(int64_t)q * mb + jj] = page;
      }
      a.dst.seq_lens[q] = r >= 0 ? a.src.seq_lens[r] : 0;
      a.dst.high_water[q] = r >= 0 ? a.src.high_water[r] : 0;
    }
    used += chunk_total;
  }
  if (threadIdx.x == 0) {
    a.dst.ctrl[BARQ_KV_CTRL_FREE_TOP] = max(0, top - used);
    atomicExch(&a.dst.ctrl[BARQ_KV_CTRL_ARRIVED], 0);
  }
  if (err) atomicOr(&a.dst.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// ---------------------------------------------------------------------------------------------
// In-place row selection with shared pages (copy-on-write beam ops) over up to kSelectPools
// pools of one geometry -- a model's layers -- per set of three launches.  New row i takes
// source row rows[i]; its blocks wholly below the source's length are shared (one more
// reference); its later blocks up to the high-water mark (the ones an append or a crop can still
// write: the "tail") are moved when i is the first new row taking that source and the page is
// held by that block alone, and copied into a page from the free stack otherwise.
//   plan   -- workgroup per pool: first new row of every source row, each new row's copy count
//             and rank (in row order), the total; if the free stack holds the copies the top
//             drops by them, else the selection is abandoned (nothing changes, POOL_EXHAUSTED).
//   build  -- workgroup (new row i, pool): shared blocks gain a reference, moved blocks keep
//             their page, copied blocks take pages top-1-rank, ... and receive the copies.  The
//             new table row, length and mark go to the pool's workspace slice.
//   settle -- workgroup (row r, pool): old row r drops its references -- except its moved tail
//             blocks, which its first taker holds on -- and a page no block holds any more is
//             pushed on the stack; then row r becomes workspace row r (rows >= n: empty).  One
//             workgroup reads and rewrites the row, so no other can race it.
// Copies are made while every source page is still held, and references are added before any is
// dropped, so a page the new rows keep never reaches zero.  Only copies need free pages: a beam
// step whose rows end in partial pages copies one page per repeated source row.
// ---------------------------------------------------------------------------------------------

constexpr int kSelectPools = 32;
constexpr int kSelectMaxBatch = 8192;  // the plan's first-taker table lives in LDS

struct SelectPool {  // the per-pool pointers of a barq_kv_pool
  const char* key_pages;
  const char* value_pages;
  int32_t* block_table;
  int32_t* seq_lens;
  int32_t* high_water;
  int32_t* free_pages;
  int32_t* ctrl;
  int32_t* page_shares;
};

struct SelectArgs {
  SelectPool pools[kSelectPools];
  int32_t num_pages[kSelectPools];
  // Pools with fp8 cold stores (cold != 0): quantised blocks are shared by reference, counted in
  // cold_shares and released to free_cold; every hot block is tail (moved or copied).
  int32_t* cold_shares[kSelectPools];
  int32_t* free_cold[kSelectPools];
  int32_t num_cold[kSelectPools];
  int32_t cold;
  const int32_t* rows;
  int32_t* ws;            // per pool, ws_pool_words: see SelectWs
  int64_t ws_pool_words;
  int64_t page_bytes;
  int32_t n;
  int32_t max_batch;
  int32_t max_blocks;
  FastDiv div_page;
};

// A pool's workspace slice: the new rows' table [n * mb], lengths [n], marks [n], copy ranks
// [n], the first taker of each old row [max_batch] (-1: not taken), the stack top before the
// copies, and whether the selection goes ahead.
struct SelectWs {
  int32_t* table;
  int32_t* lens;
  int32_t* marks;
  int32_t* rank;
  int32_t* first;
  int32_t* top;
  int32_t* go;
  __device__ SelectWs(const SelectArgs& a, int pool) {
    table = a.ws + (int64_t)pool * a.ws_pool_words;
    lens = table + (int64_t)a.n * a.max_blocks;
    marks = lens + a.n;
    rank = marks + a.n;
    first = rank + a.n;
    top = first + a.max_batch;
    go = top + 1;
  }
};

int64_t select_ws_pool_words(int64_t n, int64_t max_blocks, int64_t max_batch) {
  return n * (max_blocks + 3) + max_batch + 2;
}

// Tail of source row r: blocks [first, first + count), from the one holding seq_lens up to the
// high-water mark.
__device__ __forceinline__ void tail_blocks(const SelectPool& p, int r, int mb, const FastDiv& div_page,
                                            int* first, int* count) {
  const int nb = min(ceil_div_fd(p.high_water[r], div_page), mb);
  const int f = min((int)div_page.div((uint32_t)max(p.seq_lens[r], 0)), nb);
  *first = f;
  *count = nb - f;
}

// A block-table entry naming cold page -2 - e of a store of num_cold pages.
__device__ __forceinline__ bool cold_entry(int e, int num_cold) { return e <= -2 && -2 - e < num_cold; }

// The blocks a selection moves or copies: the tail, or, in a pool with a cold store, every block
// below the high-water mark (the cold ones among them are shared instead).
__device__ __forceinline__ void select_blocks(const SelectArgs& a, const SelectPool& p, int r, int* first,
                                              int* count) {
  tail_blocks(p, r, a.max_blocks, a.div_page, first, count);
  if (a.cold) {
    *count += *first;
    *first = 0;
  }
}

__global__ void __launch_bounds__(kThreads) select_plan_kernel(const SelectArgs a) {
  __shared__ int s_first[kSelectMaxBatch];
  __shared__ int lds_scan[kWaves];
  const SelectPool& p = a.pools[blockIdx.x];
  const int num_pages = a.num_pages[blockIdx.x];
  const SelectWs w(a, blockIdx.x);
  const int mb = a.max_blocks;
  for (int r = threadIdx.x; r < a.max_batch; r += kThreads) s_first[r] = INT_MAX;
  __syncthreads();
  for (int q = threadIdx.x; q < a.n; q += kThreads) {
    const int r = a.rows[q];
    if (r >= 0 && r < a.max_batch) atomicMin(&s_first[r], q);
  }
  __syncthreads();
  for (int r = threadIdx.x; r < a.max_batch; r += kThreads)
    w.first[r] = s_first[r] == INT_MAX ? -1 : s_first[r];
  int total = 0;
  for (int q0 = 0; q0 < a.n; q0 += kThreads) {
    const int q = q0 + (int)threadIdx.x;
    int c = 0;
    if (q < a.n) {
      const int r = a.rows[q];
      if (r >= 0 && r < a.max_batch) {
        int f, cnt;
        select_blocks(a, p, r, &f, &cnt);
        if (s_first[r] != q && !a.cold) {
          c = cnt;
        } else {
          const int ncold = a.num_cold[blockIdx.x];
          for (int t = 0; t < cnt; ++t) {
            const int e = p.block_table[(int64_t)r * mb + f + t];
            if (a.cold && cold_entry(e, ncold)) continue;  // shared
            const int page = checked_page(e, num_pages);
            c += s_first[r] != q || page < 0 || p.page_shares[page] != 0;
          }
        }
      }
    }
    int chunk_total = 0;
    const int excl = block_exclusive_scan<kWaves>(c, lds_scan, &chunk_total);
    if (q < a.n) w.rank[q] = total + excl;
    total += chunk_total;
  }
  if (threadIdx.x == 0) {
    const int top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
    const bool go = total <= top;
    *w.top = top;
    *w.go = go;
    if (go) p.ctrl[BARQ_KV_CTRL_FREE_TOP] = top - total;
    else atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], BARQ_KV_ERRBIT_POOL_EXHAUSTED);
  }
}

template <int VB>
__global__ void __launch_bounds__(kThreads) select_build_kernel(const SelectArgs a) {
  __shared__ int s_meta[6];  // source row (-1: invalid), first tail block, tails, first taker?, rank, top
  __shared__ int lds_scan[kWaves];
  __shared__ int s_copy[2 * kThreads];  // (source, destination) pages of a chunk's copies
  const SelectPool& p = a.pools[blockIdx.y];
  const int num_pages = a.num_pages[blockIdx.y];
  const SelectWs w(a, blockIdx.y);
  const int mb = a.max_blocks;
  const int i = blockIdx.x;
  if (!*w.go) return;  // uniform: the plan abandoned the selection
  if (threadIdx.x == 0) {
    const int r = a.rows[i];
    const bool valid = r >= 0 && r < a.max_batch;
    int f = 0, cnt = 0;
    if (valid) select_blocks(a, p, r, &f, &cnt);
    else atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], BARQ_KV_ERRBIT_BAD_INDEX);
    w.lens[i] = valid ? p.seq_lens[r] : 0;
    w.marks[i] = valid ? p.high_water[r] : 0;
    s_meta[0] = valid ? r : -1;
    s_meta[1] = f;
    s_meta[2] = cnt;
    s_meta[3] = valid && w.first[r] == i;
    s_meta[4] = w.rank[i];
    s_meta[5] = *w.top;
  }
  __syncthreads();
  const int r = s_meta[0], f = s_meta[1], cnt = s_meta[2], taker = s_meta[3], rank = s_meta[4], top = s_meta[5];
  const int32_t* src_row = p.block_table + (int64_t)max(r, 0) * mb;
  int32_t* dst_row = w.table + (int64_t)i * mb;
  int err = 0;
  for (int j = threadIdx.x; j < mb; j += kThreads) {
    if (j < f) {
      const int page = checked_page(src_row[j], num_pages);
      if (page >= 0) atomicAdd(&p.page_shares[page], 1);
      else err |= BARQ_KV_ERRBIT_BAD_INDEX;
      dst_row[j] = page;
    } else if (j >= f + cnt) {
      dst_row[j] = -1;
    }
  }
  // The tail, in chunks of one block per thread: moved blocks keep their page, the others take
  // the next pages of the row's range on the stack and are copied by the whole workgroup.
  const int nvec = (int)(a.page_bytes / VB);
  const int ncold = a.num_cold[blockIdx.y];
  int done = 0;
  for (int t0 = 0; t0 < cnt; t0 += kThreads) {
    const int t = t0 + (int)threadIdx.x;
    int page = -1, copy = 0;  // page: the entry kept when nothing is copied
    if (t < cnt) {
      const int e = src_row[f + t];
      if (a.cold && cold_entry(e, ncold)) {  // a quantised block never changes: shared
        page = e;
        atomicAdd(&a.cold_shares[blockIdx.y][-2 - e], 1);
      } else {
        page = checked_page(e, num_pages);
        if (page < 0) err |= BARQ_KV_ERRBIT_BAD_INDEX;
        copy = !(taker && page >= 0 && p.page_shares[page] == 0);
      }
    }
    int chunk_copies = 0;
    const int k = block_exclusive_scan<kWaves>(copy, lds_scan, &chunk_copies);
    if (t < cnt) {
      int entry = page;
      if (copy) {
        const int idx = top - 1 - (rank + done + k);
        entry = idx >= 0 ? checked_page(p.free_pages[idx], num_pages) : -1;
        if (entry < 0) err |= BARQ_KV_ERRBIT_POOL_EXHAUSTED;
        s_copy[2 * k] = page;
        s_copy[2 * k + 1] = entry;
      }
      dst_row[f + t] = entry;
    }
    __syncthreads();
    for (int c = 0; c < chunk_copies; ++c) {
      const int sp = s_copy[2 * c], dp = s_copy[2 * c + 1];
      if (sp < 0 || dp < 0) continue;
      copy_run<VB>(p.key_pages + (int64_t)sp * a.page_bytes, (char*)p.key_pages + (int64_t)dp * a.page_bytes,
                   nvec);
      copy_run<VB>(p.value_pages + (int64_t)sp * a.page_bytes,
                   (char*)p.value_pages + (int64_t)dp * a.page_bytes, nvec);
    }
    __syncthreads();
    done += chunk_copies;
  }
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

__global__ void __launch_bounds__(kThreads) select_settle_kernel(const SelectArgs a) {
  const SelectPool& p = a.pools[blockIdx.y];
  const int num_pages = a.num_pages[blockIdx.y];
  const SelectWs w(a, blockIdx.y);
  const int r = blockIdx.x;
  const int mb = a.max_blocks;
  const int n = a.n;
  if (!*w.go) return;  // uniform
  int32_t* row = p.block_table + (int64_t)r * mb;
  int f, nb;
  select_blocks(a, p, r, &f, &nb);
  nb += f;
  const int taker = w.first[r];
  const int32_t* kept = taker >= 0 ? w.table + (int64_t)taker * mb : nullptr;
  const int ncold = a.num_cold[blockIdx.y];
  int err = 0;
  for (int j = threadIdx.x; j < nb; j += kThreads) {
    const int e = row[j];
    if (a.cold && cold_entry(e, ncold)) {  // the old row's reference to a quantised block
      const int c = -2 - e;
      int32_t* shares = a.cold_shares[blockIdx.y];
      if (atomicSub(&shares[c], 1) == 0) {
        shares[c] = 0;
        const int slot = atomicAdd(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], 1);
        if (slot < ncold) a.free_cold[blockIdx.y][slot] = c;
        else err |= BARQ_KV_ERRBIT_BAD_INDEX;
      }
      continue;
    }
    const int page = checked_page(e, num_pages);
    if (page < 0) continue;
    if (kept && j >= f && kept[j] == page) continue;  // moved to its first taker
    if (atomicSub(&p.page_shares[page], 1) == 0) {
      p.page_shares[page] = 0;
      const int slot = atomicAdd(&p.ctrl[BARQ_KV_CTRL_FREE_TOP], 1);
      if (slot < num_pages) p.free_pages[slot] = page;
      else err |= BARQ_KV_ERRBIT_BAD_INDEX;
    }
  }
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
  __syncthreads();  // every read of the old row (and of its length and mark) precedes the rewrite
  for (int j = threadIdx.x; j < mb; j += kThreads) row[j] = r < n ? w.table[(int64_t)r * mb + j] : -1;
  if (threadIdx.x == 0) {
    p.seq_lens[r] = r < n ? w.lens[r] : 0;
    p.high_water[r] = r < n ? w.marks[r] : 0;
  }
}

// ---------------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------------

constexpr int64_t kI32Max = 0x7fffffffLL;

int vector_bytes(uint64_t any_bits) {
  // Largest power of two <= 16 dividing every address and byte stride OR-ed into any_bits.
  int vb = 16;
  while (vb > 1 && (any_bits & (uint64_t)(vb - 1))) vb >>= 1;
  return vb;
}

bool pool_ok(const barq_kv_pool* p) {
  if (!p || !p->key_pages || !p->value_pages || !p->block_table || !p->seq_lens ||
      !p->high_water || !p->free_pages || !p->ctrl)
    return false;
  if (p->num_pages < 1 || p->max_batch < 1 || p->max_blocks < 1 || p->page_size < 1 ||
      p->kv_heads < 1 || p->head_dim < 1)
    return false;
  if (!(p->elem_bytes == 1 || p->elem_bytes == 2 || p->elem_bytes == 4 || p->elem_bytes == 8))
    return false;
  if (p->num_pages > kI32Max || p->max_batch * p->max_blocks > kI32Max ||
      p->max_blocks * p->page_size > kI32Max)
    return false;
  if (((uintptr_t)p->ctrl) & 255u) return false;
  const int64_t tok = p->kv_heads * p->head_dim * p->elem_bytes;
  if (tok * p->page_size > kI32Max) return false;
  return true;
}

// Compute units of the current device (cached per device; 0 if the query fails).  Workgroups
// are handed to CUs round-robin, so a launch of k * CUs equal tiles gives every CU k of them.
int device_cu_count() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // 0 = not queried yet; host threads may race here
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

int launch(const void* fn, dim3 grid, void* arg, hipStream_t stream, int threads = kThreads) {
  void* args[] = {arg};
  return hipLaunchKernel(fn, grid, dim3(threads), args, 0, stream) == hipSuccess ? BARQ_KV_OK
                                                                                 : BARQ_KV_ERR_LAUNCH;
}

#define BARQ_DEFINE_VB_LAUNCH(KERNEL, ARGS)                                                     \
  int launch_##KERNEL(int vb, dim3 grid, ARGS* arg, hipStream_t stream) {                      \
    switch (vb) {                                                                               \
      case 16: return launch((const void*)&KERNEL<16>, grid, arg, stream);                     \
      case 8: return launch((const void*)&KERNEL<8>, grid, arg, stream);                       \
      case 4: return launch((const void*)&KERNEL<4>, grid, arg, stream);                       \
      case 2: return launch((const void*)&KERNEL<2>, grid, arg, stream);                       \
      default: return launch((const void*)&KERNEL<1>, grid, arg, stream);                      \
    }                                                                                           \
  }

// `rounds`: the launch's tiles run in several rounds (built for 16-byte vectors only; other
// widths take the single-round kernels).
int launch_stream_kernel(int vb, int lpp, bool rounds, dim3 grid, StreamArgs* arg, hipStream_t stream) {
#define BARQ_STREAM_CASE(VB, KERNEL, ...)                                                                 \
    switch (lpp) {                                                                                        \
      case 1: return launch((const void*)&KERNEL<VB, 1, ##__VA_ARGS__>, grid, arg, stream, kStreamThreads); \
      case 2: return launch((const void*)&KERNEL<VB, 2, ##__VA_ARGS__>, grid, arg, stream, kStreamThreads); \
      case 4: return launch((const void*)&KERNEL<VB, 4, ##__VA_ARGS__>, grid, arg, stream, kStreamThreads); \
      default: return launch((const void*)&stream_kernel_any<VB>, grid, arg, stream, kStreamThreads);     \
    }
  switch (vb) {
    case 16:
      if (rounds) {
        BARQ_STREAM_CASE(16, stream_kernel_rounds)
      } else {
        BARQ_STREAM_CASE(16, stream_kernel)
      }
    case 8: BARQ_STREAM_CASE(8, stream_kernel)
    case 4: BARQ_STREAM_CASE(4, stream_kernel)
    case 2: BARQ_STREAM_CASE(2, stream_kernel)
    default: BARQ_STREAM_CASE(1, stream_kernel)
  }
#undef BARQ_STREAM_CASE
}

template <bool BAL>
int launch_lean_kernel(int nu, int lpp, dim3 grid, StreamArgs* arg, hipStream_t stream) {
#define BARQ_LEAN_FN(NU, L) (BAL ? (const void*)&lean_balanced_kernel<NU, L> : (const void*)&lean_stream_kernel<NU, L>)
#define BARQ_LEAN_CASE(NU)                                                                 \
    switch (lpp) {                                                                          \
      case 1: return launch(BARQ_LEAN_FN(NU, 1), grid, arg, stream, kStreamThreads);        \
      case 2: return launch(BARQ_LEAN_FN(NU, 2), grid, arg, stream, kStreamThreads);        \
      default: return launch(BARQ_LEAN_FN(NU, 4), grid, arg, stream, kStreamThreads);       \
    }
  switch (nu) {
    case 4: BARQ_LEAN_CASE(4)
    case 8: BARQ_LEAN_CASE(8)
    default: BARQ_LEAN_CASE(16)
  }
#undef BARQ_LEAN_CASE
#undef BARQ_LEAN_FN
}

int launch_known_kernel(int nu, int lpp, dim3 grid, StreamArgs* arg, const KnownState* known, hipStream_t stream) {
  const void* fn = nullptr;
#define BARQ_KNOWN_CASE(NU)                                              \
  switch (lpp) {                                                         \
    case 1: fn = (const void*)&lean_known_kernel<NU, 1>; break;          \
    case 2: fn = (const void*)&lean_known_kernel<NU, 2>; break;          \
    default: fn = (const void*)&lean_known_kernel<NU, 4>; break;         \
  }
  switch (nu) {
    case 4: BARQ_KNOWN_CASE(4) break;
    case 8: BARQ_KNOWN_CASE(8) break;
    default: BARQ_KNOWN_CASE(16) break;
  }
#undef BARQ_KNOWN_CASE
  KnownState ks = *known;
  void* args[] = {arg, &ks};
  return hipLaunchKernel(fn, grid, dim3(kStreamThreads), args, 0, stream) == hipSuccess ? BARQ_KV_OK
                                                                                      : BARQ_KV_ERR_LAUNCH;
}

BARQ_DEFINE_VB_LAUNCH(dense_append_kernel, DenseArgs)
BARQ_DEFINE_VB_LAUNCH(copy_rows_kernel, CopyArgs)
BARQ_DEFINE_VB_LAUNCH(select_build_kernel, SelectArgs)

// Shared body of append / gather / update.
int run_stream(const barq_kv_pool* pool, const void* ks, const void* vs, int64_t batch,
               int64_t tokens, int64_t sb, int64_t sh, int64_t st, void* ko, void* vo,
               int64_t seq_out, int64_t osb, int64_t osh, int64_t oss, int64_t flags,
               bool gather, void* stream, const KnownState* known = nullptr) {
  if (!pool_ok(pool)) return BARQ_KV_ERR_INVALID;
  if (batch < 0 || batch > pool->max_batch || tokens < 0 || tokens > kI32Max) return BARQ_KV_ERR_INVALID;
  if (flags & ~(int64_t)(BARQ_KV_SEQ_FROM_DEVICE | BARQ_KV_SEPARATE_FINALIZE)) return BARQ_KV_ERR_INVALID;
  const int64_t cap = pool->max_blocks * pool->page_size;
  if (gather && (seq_out < 0 || seq_out > cap)) return BARQ_KV_ERR_INVALID;
  if (tokens > cap) return BARQ_KV_ERR_INVALID;
  if (batch == 0) return BARQ_KV_OK;
  // An update's tiles cover output positions only, so the output must reach the new tokens.
  if (gather && tokens > seq_out) return BARQ_KV_ERR_INVALID;
  if (tokens == 0 && (!gather || seq_out == 0)) return BARQ_KV_OK;
  if (tokens > 0 && (!ks || !vs || sb < 0 || sh < 0 || st < 0)) return BARQ_KV_ERR_INVALID;
  if (gather && (!ko || !vo || osb < 0 || osh < 0 || oss < 0)) return BARQ_KV_ERR_INVALID;

  const int64_t eb = pool->elem_bytes;
  const int64_t row_bytes = pool->head_dim * eb;
  const int64_t tok_bytes = pool->kv_heads * row_bytes;
  uint64_t bits = (uint64_t)row_bytes | (uint64_t)(uintptr_t)pool->key_pages |
                  (uint64_t)(uintptr_t)pool->value_pages;
  if (tokens > 0) bits |= (uint64_t)(uintptr_t)ks | (uint64_t)(uintptr_t)vs | (uint64_t)(sb * eb) |
                          (uint64_t)(sh * eb) | (uint64_t)(st * eb);
  if (gather) bits |= (uint64_t)(uintptr_t)ko | (uint64_t)(uintptr_t)vo | (uint64_t)(osb * eb) |
                      (uint64_t)(osh * eb) | (uint64_t)(oss * eb);
  const int vb = vector_bytes(bits);
  const int64_t vr = row_bytes / vb;
  const int64_t hv = pool->kv_heads * vr;

  const int64_t P = pool->page_size;
  const int64_t span = gather ? seq_out : tokens;
  // The wave-uniform mapping needs whole 64-vector runs per wave and 32-bit offsets within a
  // page, within a row's output ([seq_out, H, D] span) and within a row's input.
  const auto span32 = [](int64_t n, int64_t stride, int64_t inner) {
    return stride >= 0 && stride <= (int64_t)UINT32_MAX && (n - 1) * stride + inner <= (int64_t)UINT32_MAX;
  };
  const int64_t head_span_out = (pool->kv_heads - 1) * osh * eb + row_bytes;
  const int64_t head_span_in = (pool->kv_heads - 1) * sh * eb + row_bytes;
  const bool fast = (hv == 64 || hv == 128 || hv == 256) && P * tok_bytes <= (int64_t)UINT32_MAX &&
                    (!gather || (osh * eb <= (int64_t)UINT32_MAX && span32(seq_out, oss * eb, head_span_out))) &&
                    (tokens == 0 || (sh * eb <= (int64_t)UINT32_MAX && span32(tokens, st * eb, head_span_in)));
  const int64_t ncu = device_cu_count();

  // Lean kernel: a gather launch whose tiles of one page -- else two -- are all resident at once.
  const int64_t lpp = hv / 64;
  // Balanced lean tiles: every (row, K or V) cut into m equal chunks of at most a page's
  // positions, 2 * batch * m the smallest multiple of the CU count, up to per_cu tiles per CU,
  // that holds the one-page tiles' chunks; 0 if none does.
  // (C2, context 513-576: 15.2 -> 14.1 us per launch.)  Two-page tiles stay page-aligned: cut
  // the same way (up to three blocks a tile) they ran 1-2 % slower; six balanced one-page tiles
  // per CU instead of two-page ones, 20 % slower; balanced chunks of up to two pages, three or
  // four per CU, in place of the one-page tiles (C2 at extents 576 / 640): 14.84 / 16.02 ->
  // 15.28 / 16.22 and 17.52 / 17.57 us.
  const auto balanced_chunks = [&](int64_t aligned, int64_t per_cu) -> int64_t {
    for (int64_t k = 1; k <= per_cu; ++k)
      if ((k * ncu) % (2 * batch) == 0 && k * ncu / (2 * batch) >= aligned) return k * ncu / (2 * batch);
    return 0;
  };
  int64_t lean_ppt = 0, lean_nu = 0, lean_m = 0;
  if (gather && fast && vb == 16 && batch <= kWave && ncu > 0) {
    for (int64_t q = 1; q <= 2 && lean_ppt == 0; ++q) {
      if ((q * P * lpp) % 4 != 0) continue;  // whole steps of 4 / LPP positions
      const int64_t nu = q * P * lpp / 4;
      if (nu != 4 && nu != 8 && nu != 16) continue;
      const int64_t resident = nu == 16 ? kLeanResidentTilesPerCU16 : kLeanResidentTilesPerCU;
      const int64_t aligned = (span + q * P - 1) / (q * P);
      if (2 * batch * aligned <= resident * ncu) {
        lean_ppt = q;
        lean_nu = nu;
        // one-page tiles, at least one per CU, not a multiple of the CU count: balance them
        if (q == 1 && 2 * batch * aligned >= ncu && (2 * batch * aligned) % ncu != 0)
          lean_m = balanced_chunks(aligned, resident);
      }
    }
  }

  // Positions per tile: whole pages, about kTileTargetBytes of each of K and V.
  int64_t pages_per_tile = kTileTargetBytes / (P * tok_bytes);
  if (pages_per_tile < 1) pages_per_tile = 1;
  if (pages_per_tile > kMaxTilePages) pages_per_tile = kMaxTilePages;
  // An append tile starts at an arbitrary slot, so its `chunk` positions touch at most
  // pages_per_tile + 1 blocks: s_pbase holds kMaxTilePages + 1.
  if (pages_per_tile > 1 && 2 * batch * ((span + pages_per_tile * P - 1) / (pages_per_tile * P)) > kLargeLaunchTiles)
    pages_per_tile /= 2;
  if (lean_ppt > 0) pages_per_tile = lean_ppt;
  const int64_t chunk = pages_per_tile * P;
  if (chunk * hv > kI32Max - (int64_t)kThreads * kUnroll) return BARQ_KV_ERR_INVALID;
  int64_t chunks = (span + chunk - 1) / chunk;
  if (lean_m > 0) chunks = lean_m;
  const int64_t tiles = 2 * batch * chunks;
  if (tiles > kI32Max) return BARQ_KV_ERR_INVALID;

  // A gather launch of the control-wave kernel whose tiles are all resident at once ends when the
  // CUs holding the most tiles finish (a CU streams at a roughly fixed rate).  When the tile
  // count is not a multiple of the CU count, whole rounds of tiles are kept and the remaining
  // positions of every (row, K or V) are cut into pieces, one per CU in total: every CU then
  // gets the same work.
  const int64_t rk = 2 * batch;  // (row, K or V) streams
  int64_t full_tiles = tiles, tail_lo = 0, piece_len = 1, per_rk = 1, grid = tiles;
  if (gather && fast && lean_ppt == 0) {
    if (ncu > 0 && ncu % rk == 0 && tiles > ncu && tiles % ncu != 0 && tiles <= kResidentTilesPerCU * ncu) {
      per_rk = ncu / rk;
      const int64_t full_chunks = (tiles / ncu) * per_rk;  // whole rounds of tiles
      tail_lo = full_chunks * chunk;
      piece_len = (span - tail_lo + per_rk - 1) / per_rk;  // <= chunk
      full_tiles = rk * full_chunks;
      grid = full_tiles + ncu;
    }
  }

  StreamArgs a;
  a.pool = *pool;
  a.in_k = (const char*)ks;
  a.in_v = (const char*)vs;
  a.out_k = (char*)ko;
  a.out_v = (char*)vo;
  a.in_sb = sb * eb;
  a.in_sh = sh * eb;
  a.in_st = st * eb;
  a.out_sb = osb * eb;
  a.out_sh = osh * eb;
  a.out_ss = oss * eb;
  a.page_bytes = P * tok_bytes;
  a.tok_bytes = tok_bytes;
  a.batch = (int32_t)batch;
  a.tokens = (int32_t)tokens;
  a.seq_out = (int32_t)(gather ? seq_out : 0);
  a.chunk = (int32_t)chunk;
  a.ppt = (int32_t)pages_per_tile;
  a.gather = gather ? 1 : 0;
  a.seq_from_device = (gather && (flags & BARQ_KV_SEQ_FROM_DEVICE)) ? 1 : 0;
  a.commit_in_kernel = (flags & BARQ_KV_SEPARATE_FINALIZE) ? 0 : 1;
  a.hv = (int32_t)hv;
  a.nsub = (int32_t)std::min<int64_t>(grid, BARQ_KV_CTRL_SUBCOUNTERS);
  a.div_hv = FastDiv::make((uint32_t)hv);
  a.div_vr = FastDiv::make((uint32_t)vr);
  a.div_page = FastDiv::make((uint32_t)P);
  a.div_chunks = FastDiv::make((uint32_t)(full_tiles / rk));  // chunks per (row, K or V) in full tiles
  a.full_tiles = (int32_t)full_tiles;
  a.tail_lo = (int32_t)tail_lo;
  a.piece_len = (int32_t)piece_len;
  a.div_pieces = FastDiv::make((uint32_t)per_rk);

  hipStream_t s = (hipStream_t)stream;
  // Launches with more tiles than the CUs hold at once take the kernel built for several rounds.
  const bool rounds = fast && ncu > 0 && grid > kResidentTilesPerCU * ncu;
  // The caller's row state in the arguments: page-aligned lean launches of an append and gather
  // whose extent is given (the per-call path of an eager caller).
  if (known && lean_ppt > 0 && lean_m == 0 && tokens > 0 && a.commit_in_kernel && !a.seq_from_device)
    return launch_known_kernel((int)lean_nu, (int)lpp, dim3((uint32_t)grid), &a, known, s);
  int rc = lean_ppt > 0 ? (lean_m > 0 ? launch_lean_kernel<true>((int)lean_nu, (int)lpp, dim3((uint32_t)grid), &a, s)
                                      : launch_lean_kernel<false>((int)lean_nu, (int)lpp, dim3((uint32_t)grid), &a, s))
                        : launch_stream_kernel(vb, fast ? (int)(hv / 64) : 0, rounds, dim3((uint32_t)grid), &a, s);
  if (rc != BARQ_KV_OK) return rc;
  if (tokens > 0 && !a.commit_in_kernel) {
    barq_kv_pool pc = *pool;
    int32_t b32 = (int32_t)batch, t32 = (int32_t)tokens;
    int32_t limit = gather ? a.seq_out : INT_MAX;
    FastDiv dp = a.div_page;
    void* args[] = {&pc, &b32, &t32, &limit, &dp};
    if (hipLaunchKernel((const void*)&commit_kernel, dim3(1), dim3(kThreads), args, 0, s) != hipSuccess)
      return BARQ_KV_ERR_LAUNCH;
  }
  return BARQ_KV_OK;
}

// barq_kv_select_rows_layers, and with `colds` (one per pool) its cold-store form.
int select_rows_impl(const barq_kv_pool* pools, const barq_kv_cold* colds, int64_t num_pools,
                     const int32_t* src_rows, int64_t num_rows, int32_t* workspace, int64_t workspace_words,
                     void* stream) {
  if (!pools || num_pools < 1) return BARQ_KV_ERR_INVALID;
  const barq_kv_pool& g = pools[0];
  for (int64_t l = 0; l < num_pools; ++l) {
    const barq_kv_pool& p = pools[l];
    if (!pool_ok(&p) || !p.page_shares || p.num_pages > kI32Max) return BARQ_KV_ERR_INVALID;
    if (p.max_batch != g.max_batch || p.max_blocks != g.max_blocks || p.page_size != g.page_size ||
        p.kv_heads != g.kv_heads || p.head_dim != g.head_dim || p.elem_bytes != g.elem_bytes)
      return BARQ_KV_ERR_INVALID;
    for (int64_t m = 0; m < l; ++m)  // a pool named twice would release its rows twice
      if (pools[m].block_table == p.block_table || pools[m].ctrl == p.ctrl || pools[m].page_shares == p.page_shares)
        return BARQ_KV_ERR_INVALID;
    if (colds) {
      const barq_kv_cold& c = colds[l];
      if (!c.cold_shares || !c.free_cold || c.num_cold < 1 || c.num_cold >= kI32Max - 2) return BARQ_KV_ERR_INVALID;
      for (int64_t m = 0; m < l; ++m)
        if (colds[m].cold_shares == c.cold_shares || colds[m].free_cold == c.free_cold) return BARQ_KV_ERR_INVALID;
    }
  }
  if (num_rows < 0 || num_rows > g.max_batch || g.max_batch > kSelectMaxBatch || g.max_blocks > kI32Max)
    return BARQ_KV_ERR_INVALID;
  const int64_t ws_pool_words = select_ws_pool_words(num_rows, g.max_blocks, g.max_batch);
  if ((num_rows > 0 && !src_rows) || !workspace ||
      workspace_words < std::min<int64_t>(num_pools, kSelectPools) * ws_pool_words)
    return BARQ_KV_ERR_INVALID;
  SelectArgs a;
  a.rows = src_rows;
  a.ws = workspace;
  a.ws_pool_words = ws_pool_words;
  a.page_bytes = g.page_size * g.kv_heads * g.head_dim * g.elem_bytes;
  a.n = (int32_t)num_rows;
  a.max_batch = (int32_t)g.max_batch;
  a.max_blocks = (int32_t)g.max_blocks;
  a.div_page = FastDiv::make((uint32_t)g.page_size);
  a.cold = colds ? 1 : 0;
  hipStream_t s = (hipStream_t)stream;
  int rc = BARQ_KV_OK;
  for (int64_t l0 = 0; l0 < num_pools && rc == BARQ_KV_OK; l0 += kSelectPools) {
    const int set = (int)std::min<int64_t>(kSelectPools, num_pools - l0);
    uint64_t bits = (uint64_t)a.page_bytes;
    for (int k = 0; k < kSelectPools; ++k) {
      const barq_kv_pool& p = pools[l0 + std::min(k, set - 1)];
      a.pools[k] = SelectPool{(const char*)p.key_pages, (const char*)p.value_pages, p.block_table, p.seq_lens,
                              p.high_water, p.free_pages, p.ctrl, p.page_shares};
      a.num_pages[k] = (int32_t)p.num_pages;
      const barq_kv_cold* c = colds ? &colds[l0 + std::min(k, set - 1)] : nullptr;
      a.cold_shares[k] = c ? c->cold_shares : nullptr;
      a.free_cold[k] = c ? c->free_cold : nullptr;
      a.num_cold[k] = c ? (int32_t)c->num_cold : 0;
      bits |= (uint64_t)(uintptr_t)p.key_pages | (uint64_t)(uintptr_t)p.value_pages;
    }
    rc = launch((const void*)&select_plan_kernel, dim3((uint32_t)set), &a, s);
    if (rc == BARQ_KV_OK && num_rows > 0)
      rc = launch_select_build_kernel(vector_bytes(bits), dim3((uint32_t)num_rows, (uint32_t)set), &a, s);
    if (rc == BARQ_KV_OK)
      rc = launch((const void*)&select_settle_kernel, dim3((uint32_t)g.max_batch, (uint32_t)set), &a, s);
  }
  return rc;
}

}  // namespace

extern "C" {

const char* barq_kv_version(void) { return "barq_kv 0.1.0 gfx950"; }

const char* barq_kv_status_string(int status) {
  switch (status) {
    case BARQ_KV_OK: return "ok";
    case BARQ_KV_ERR_INVALID: return "invalid argument (pointer, size, stride or alignment)";
    case BARQ_KV_ERR_LAUNCH: return "HIP kernel launch failed";
    case BARQ_KV_ERR_SCRATCH: return "request exceeds the static scratch (BARQ_KV_SCRATCH_BYTES per GPU)";
    default: return "unknown status";
  }
}

int barq_kv_append_dense(void* key_cache, void* value_cache, int32_t* seq_lens,
                         const void* key_states, const void* value_states, int64_t batch,
                         int64_t kv_heads, int64_t tokens, int64_t head_dim, int64_t cache_batch,
                         int64_t max_blocks, int64_t page_size, int64_t elem_bytes,
                         int64_t stride_b, int64_t stride_h, int64_t stride_t, void* stream) {
  if (!key_cache || !value_cache || !seq_lens) return BARQ_KV_ERR_INVALID;
  if (batch < 0 || kv_heads < 1 || tokens < 0 || head_dim < 1 || max_blocks < 1 || page_size < 1)
    return BARQ_KV_ERR_INVALID;
  if (batch > cache_batch) return BARQ_KV_ERR_INVALID;
  if (!(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8)) return BARQ_KV_ERR_INVALID;
  if (batch == 0) return BARQ_KV_OK;
  hipStream_t s = (hipStream_t)stream;
  if (tokens > 0) {
    if (!key_states || !value_states) return BARQ_KV_ERR_INVALID;
    const int64_t row_bytes = head_dim * elem_bytes;
    const uint64_t bits = (uint64_t)row_bytes | (uint64_t)(uintptr_t)key_cache |
                          (uint64_t)(uintptr_t)value_cache | (uint64_t)(uintptr_t)key_states |
                          (uint64_t)(uintptr_t)value_states | (uint64_t)(stride_b * elem_bytes) |
                          (uint64_t)(stride_h * elem_bytes) | (uint64_t)(stride_t * elem_bytes);
    const int vb = vector_bytes(bits);
    const int64_t vr = row_bytes / vb;
    const int64_t total = batch * kv_heads * tokens * vr;
    if (total > kI32Max || max_blocks * page_size > kI32Max) return BARQ_KV_ERR_INVALID;
    DenseArgs a;
    a.kc = (char*)key_cache;
    a.vc = (char*)value_cache;
    a.seq_lens = seq_lens;
    a.ks = (const char*)key_states;
    a.vs = (const char*)value_states;
    a.sb = stride_b * elem_bytes;
    a.sh = stride_h * elem_bytes;
    a.st = stride_t * elem_bytes;
    a.row_bytes = row_bytes;
    a.heads = (int32_t)kv_heads;
    a.tokens = (int32_t)tokens;
    a.max_blocks = (int32_t)max_blocks;
    a.page_size = (int32_t)page_size;
    a.total = (int32_t)total;
    a.div_vr = FastDiv::make((uint32_t)vr);
    a.div_tokens = FastDiv::make((uint32_t)tokens);
    a.div_heads = FastDiv::make((uint32_t)kv_heads);
    a.div_page = FastDiv::make((uint32_t)page_size);
    int64_t blocks = (total + (int64_t)kThreads * kUnroll - 1) / ((int64_t)kThreads * kUnroll);
    if (blocks > 65536) blocks = 65536;
    const int rc = launch_dense_append_kernel(vb, dim3((uint32_t)blocks), &a, s);
    if (rc != BARQ_KV_OK) return rc;
  }
  int32_t b32 = (int32_t)batch, t32 = (int32_t)tokens;
  void* args[] = {&seq_lens, &b32, &t32};
  if (hipLaunchKernel((const void*)&dense_bump_kernel, dim3((uint32_t)((batch + kThreads - 1) / kThreads)),
                      dim3(kThreads), args, 0, s) != hipSuccess)
    return BARQ_KV_ERR_LAUNCH;
  return BARQ_KV_OK;
}

int barq_kv_pool_reset(const barq_kv_pool* pool, const int32_t* page_order, void* stream) {
  if (!pool_ok(pool)) return BARQ_KV_ERR_INVALID;
  barq_kv_pool p = *pool;
  const int64_t n = std::max(std::max(p.num_pages, p.max_batch * p.max_blocks),
                             (int64_t)BARQ_KV_CTRL_WORDS);
  int64_t blocks = (n + kThreads - 1) / kThreads;
  if (blocks > 4096) blocks = 4096;
  const int32_t* order = page_order;
  void* args[] = {&p, &order};
  return hipLaunchKernel((const void*)&reset_kernel, dim3((uint32_t)blocks), dim3(kThreads), args, 0,
                         (hipStream_t)stream) == hipSuccess
             ? BARQ_KV_OK
             : BARQ_KV_ERR_LAUNCH;
}

int barq_kv_append(const barq_kv_pool* pool, const void* key_states, const void* value_states,
                   int64_t batch, int64_t tokens, int64_t stride_b, int64_t stride_h,
                   int64_t stride_t, void* stream) {
  return run_stream(pool, key_states, value_states, batch, tokens, stride_b, stride_h, stride_t,
                    nullptr, nullptr, 0, 0, 0, 0, 0, false, stream);
}

int barq_kv_gather(const barq_kv_pool* pool, void* key_out, void* value_out, int64_t batch,
                   int64_t seq_out, int64_t out_stride_b, int64_t out_stride_h,
                   int64_t out_stride_s, int64_t flags, void* stream) {
  return run_stream(pool, nullptr, nullptr, batch, 0, 0, 0, 0, key_out, value_out, seq_out,
                    out_stride_b, out_stride_h, out_stride_s, flags, true, stream);
}

int barq_kv_update(const barq_kv_pool* pool, const void* key_states, const void* value_states,
                   int64_t batch, int64_t tokens, int64_t stride_b, int64_t stride_h,
                   int64_t stride_t, void* key_out, void* value_out, int64_t seq_out,
                   int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_s,
                   int64_t flags, void* stream) {
  return run_stream(pool, key_states, value_states, batch, tokens, stride_b, stride_h, stride_t,
                    key_out, value_out, seq_out, out_stride_b, out_stride_h, out_stride_s, flags,
                    true, stream);
}

int barq_kv_update_known(const barq_kv_pool* pool, const void* key_states, const void* value_states,
                         int64_t batch, int64_t tokens, int64_t stride_b, int64_t stride_h,
                         int64_t stride_t, void* key_out, void* value_out, int64_t seq_out,
                         int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_s,
                         const int32_t* seq_lens, const int32_t* high_water, int64_t free_top,
                         void* stream) {
  if (batch < 0 || (batch > 0 && (!seq_lens || !high_water)) || free_top < 0 ||
      (pool && free_top > pool->num_pages))
    return BARQ_KV_ERR_INVALID;
  if (batch > kWave)  // the kernel's commit holds one row per lane: the device-read path
    return run_stream(pool, key_states, value_states, batch, tokens, stride_b, stride_h, stride_t,
                      key_out, value_out, seq_out, out_stride_b, out_stride_h, out_stride_s, 0, true, stream);
  KnownState known;
  for (int64_t r = 0; r < kWave; ++r) {
    known.len[r] = r < batch ? seq_lens[r] : 0;
    known.hw[r] = r < batch ? high_water[r] : 0;
    if (r < batch && (known.len[r] < 0 || known.hw[r] < known.len[r])) return BARQ_KV_ERR_INVALID;
  }
  known.top = (int32_t)free_top;
  return run_stream(pool, key_states, value_states, batch, tokens, stride_b, stride_h, stride_t,
                    key_out, value_out, seq_out, out_stride_b, out_stride_h, out_stride_s, 0,
                    true, stream, &known);
}

int barq_kv_crop(const barq_kv_pool* pool, int64_t batch, int64_t max_length, void* stream) {
  if (!pool_ok(pool) || batch < 0 || batch > pool->max_batch || max_length < 0) return BARQ_KV_ERR_INVALID;
  if (batch == 0) return BARQ_KV_OK;
  int32_t* lens = pool->seq_lens;
  int32_t b32 = (int32_t)batch;
  int32_t m32 = (int32_t)std::min(max_length, kI32Max);
  void* args[] = {&lens, &b32, &m32};
  return hipLaunchKernel((const void*)&crop_kernel, dim3((uint32_t)((batch + kThreads - 1) / kThreads)),
                         dim3(kThreads), args, 0, (hipStream_t)stream) == hipSuccess
             ? BARQ_KV_OK
             : BARQ_KV_ERR_LAUNCH;
}

int barq_kv_free_rows(const barq_kv_pool* pool, const int32_t* rows, int64_t num_rows,
                      void* stream) {
  if (!pool_ok(pool) || num_rows < 0 || num_rows > pool->max_batch) return BARQ_KV_ERR_INVALID;
  if (num_rows == 0) return BARQ_KV_OK;
  if (!rows) return BARQ_KV_ERR_INVALID;
  barq_kv_pool p = *pool;
  int32_t n32 = (int32_t)num_rows;
  FastDiv dp = FastDiv::make((uint32_t)p.page_size);
  void* args[] = {&p, &rows, &n32, &dp};
  return hipLaunchKernel((const void*)&free_rows_kernel, dim3(1), dim3(kThreads), args, 0,
                         (hipStream_t)stream) == hipSuccess
             ? BARQ_KV_OK
             : BARQ_KV_ERR_LAUNCH;
}

int64_t barq_kv_select_workspace_words(const barq_kv_pool* pool, int64_t num_pools, int64_t num_rows) {
  if (!pool_ok(pool) || num_pools < 1 || num_rows < 0 || num_rows > pool->max_batch ||
      pool->max_batch > kSelectMaxBatch)
    return -1;
  return std::min<int64_t>(num_pools, kSelectPools) *
         select_ws_pool_words(num_rows, pool->max_blocks, pool->max_batch);
}

int barq_kv_select_rows_layers(const barq_kv_pool* pools, int64_t num_pools, const int32_t* src_rows,
                               int64_t num_rows, int32_t* workspace, int64_t workspace_words,
                               void* stream) {
  return select_rows_impl(pools, nullptr, num_pools, src_rows, num_rows, workspace, workspace_words, stream);
}

int barq_kv_select_rows_cold_layers(const barq_kv_pool* pools, const barq_kv_cold* colds, int64_t num_pools,
                                    const int32_t* src_rows, int64_t num_rows, int32_t* workspace,
                                    int64_t workspace_words, void* stream) {
  if (!colds) return BARQ_KV_ERR_INVALID;
  return select_rows_impl(pools, colds, num_pools, src_rows, num_rows, workspace, workspace_words, stream);
}

int barq_kv_select_rows(const barq_kv_pool* pool, const int32_t* src_rows, int64_t num_rows,
                        int32_t* workspace, int64_t workspace_words, void* stream) {
  return barq_kv_select_rows_layers(pool, 1, src_rows, num_rows, workspace, workspace_words, stream);
}

int barq_kv_copy_rows(const barq_kv_pool* src, const barq_kv_pool* dst, const int32_t* src_rows,
                      int64_t num_rows, void* stream) {
  if (!pool_ok(src) || !pool_ok(dst)) return BARQ_KV_ERR_INVALID;
  if (src->page_size != dst->page_size || src->kv_heads != dst->kv_heads ||
      src->head_dim != dst->head_dim || src->elem_bytes != dst->elem_bytes ||
      src->max_blocks != dst->max_blocks)
    return BARQ_KV_ERR_INVALID;
  if (num_rows < 0 || num_rows > dst->max_batch) return BARQ_KV_ERR_INVALID;
  if (num_rows == 0) return BARQ_KV_OK;
  if (!src_rows) return BARQ_KV_ERR_INVALID;
  const int64_t tiles = num_rows * src->max_blocks;
  if (tiles > kI32Max) return BARQ_KV_ERR_INVALID;
  CopyArgs a;
  a.src = *src;
  a.dst = *dst;
  a.rows = src_rows;
  a.n = (int32_t)num_rows;
  a.page_bytes = src->page_size * src->kv_heads * src->head_dim * src->elem_bytes;
  a.div_page = FastDiv::make((uint32_t)src->page_size);
  a.div_blocks = FastDiv::make((uint32_t)src->max_blocks);
  const uint64_t bits = (uint64_t)a.page_bytes | (uint64_t)(uintptr_t)src->key_pages |
                        (uint64_t)(uintptr_t)src->value_pages | (uint64_t)(uintptr_t)dst->key_pages |
                        (uint64_t)(uintptr_t)dst->value_pages;
  return launch_copy_rows_kernel(vector_bytes(bits), dim3((uint32_t)tiles), &a, (hipStream_t)stream);
}

}  // extern "C"
