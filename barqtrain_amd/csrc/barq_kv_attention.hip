// Decode attention that reads K and V straight from the page pool through the block table
// (the "attention reads" of a paged cache), for MI355X (gfx950), behind include/barq_kv.h.
//
//   out[b, h, i, :] = softmax_t(scale * q[b, h, i, :] . K[b, h / G, t, :]) V[b, h / G, t, :]
//   over the positions t <= seq_lens[b] - T + i of row b (the row's own length, causal over the
//   T new query tokens), G = q_heads / kv_heads (grouped-query attention).
//
// Work split (flash decoding over a flat schedule): the launch has one single-wave workgroup per
// resident wave slot of the GPU.  All (row, kv head) pairs' positions, in 16-position chunks,
// form one row-major list; it is cut into equal ranges of chunks, one range per wave (or several,
// grid-stride, when the caller fixes a smaller range).  Every wave therefore streams the same
// number of bytes and every CU carries the same load, whatever the rows' lengths.  A wave walks
// its range pair by pair ("pieces"), streaming each piece's chunks with the next chunk's loads in
// flight while the current one is computed.  The G*T query rows of a kv head share every K/V byte
// the wave loads, so each byte of the pages is read once per launch.
//
// Per piece: the block-table entries (one per lane, a sliding window of kTableEntries blocks)
// give the page bases by readlane (scalar) or ds_bpermute (per lane, odd page sizes).  Scores
// come from the bf16/fp16 16x16x32 MFMA (query rows padded to 16, the chunk's positions as the
// 16 columns).  P.V runs on the fp32 4x4x1 MFMA in 16 blocks: a lane's 16-byte load of V holds 8
// consecutive head dims of one position, and element e of it is the lane's B operand of the e-th
// MFMA, so V is consumed in the layout it is stored in (no transpose, no LDS staging of V) and
// the probabilities stay fp32.  Online softmax per query row (running max / sum, base-2).
// A piece that is a whole pair writes the output; otherwise it writes a partial record, merged
// by a second launch (the launch boundary makes the records visible: no fences, no counters).
// Piece (range r, pair p) owns record r + p: along the schedule r and p never decrease, so no
// two pieces share a record.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <type_traits>

#include "barq_kv.h"
#include "barq_kv_fp8.h"
#include "fastdiv.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kBlock = 16;                 // positions per chunk: one score MFMA's columns
constexpr int kMaxRows = 16;               // query rows (G * T) one wave serves
constexpr int kThreads = 256;              // workgroup of the merge kernel ...
constexpr int kMergeWide = 1024;           // ... or this, for grids of fewer workgroups than
constexpr int kMergeWideBelow = 256;       // this (the CUs of an MI355X)
constexpr int kTableRegs = 4;              // block-table window: lanes x registers
constexpr int kTableEntries = kTableRegs * 64;
constexpr int kMaxBatch = 1024;            // rows whose lengths the schedule stages in LDS
constexpr int kMaxWaves = 2048;            // resident waves of an MI355X: 256 CUs x 4 SIMDs x 2
constexpr int kMinRangeChunks = 4;         // the automatic range never goes below 64 positions
constexpr int kPairWaves = 8;              // waves of a pair-kernel workgroup
// The pair kernel (one workgroup per (row, kv head) pair) takes launches of at most kPairMaxChunks
// 16-position chunks a pair (max_seq); from kPairMinPairs pairs with up to 4 query rows at most
// kPairMaxChunksR1, and over two-byte pages from twice the pairs (every CU busy)
// kPairMaxChunksR1Wide.
constexpr int64_t kPairMinPairs = 128;
constexpr int64_t kPairMaxChunks = 44;
constexpr int64_t kPairMaxChunksR1 = 64;
constexpr int64_t kPairMaxChunksR1Wide = 128;
static_assert(kPairMaxChunks <= kTableEntries && kPairMaxChunksR1Wide <= kTableEntries,
              "a pair's blocks fit one table window");
// When several workgroups a pair fit on the GPU at once (C2: 128 pairs, 256 CUs: two), a pair is
// cut over as many of them as give each at least pair_part_chunks<R>() chunks, at most kMaxSplit
// (the exchange costs ~1.3 us; shorter parts lose more than they gain: at the C2 shape two
// workgroups break even at ~18-22 chunks with 4 query rows, ~27 with 8).  With three or more a
// pair, rows of up to kSplitChunksPerPart chunks a workgroup take the pair kernel.
template <int R>
__host__ __device__ constexpr int pair_part_chunks() {
  return R == 1 ? 11 : 14;
}
constexpr int kMaxSplit = 8;
constexpr int64_t kSplitChunksPerPart = 24;
constexpr int kSplitAny = 0;  // attention_pair_kernel's S: the grid's count, 3 .. kMaxSplit
// Longer rows at small batches (C4: one row of 32k positions, 8 pairs): up to kMaxSplitLong
// workgroups a pair, past 8 parts at least kLongPartChunks chunks each and at most
// kLongChunksPerPart (a part's blocks fit one table window, loaded at the part's start).
constexpr int kSplitLong = -1;  // attention_pair_kernel's S: the grid's count, 3 .. kMaxSplitLong
constexpr int kMaxSplitLong = 32;
constexpr int kLongPartChunks = 32;
constexpr int64_t kLongChunksPerPart = 72;

enum : int { kBF16 = 0, kF16 = 1 };

// Head sizes the kernels are built for (HD = 64, 128, and 256 on two-byte pages through the flat
// schedule at one wave per SIMD) and the lane layout each gives.  Scores:
// lane (g, n16) of the 16x16x32 MFMA holds dims 32 * step + 8 * g .. +7 of one position, HD / 32
// steps.  V: a position's HD dims are HD / 8 lanes of 8 dims, so one 16-byte load per lane covers
// 64 / (HD / 8) positions and a chunk takes 16 / that many loads.
template <int HD>
struct Head {
  static_assert(HD == 64 || HD == 128 || HD == 256, "head sizes 64, 128 and 256");
  static constexpr int kSteps = HD / 32;              // k-steps of the score MFMA
  static constexpr int kVLanes = HD / 8;              // lanes of one position's V
  static constexpr int kVPos = kWave / kVLanes;       // positions of one V load
  static constexpr int kVLoads = kBlock / kVPos;      // V loads of one chunk
};

struct AttnArgs {
  const char* kpages;
  const char* vpages;
  const int32_t* block_table;
  const int32_t* seq_lens;
  int32_t* errors;
  int32_t* ctrl;        // the pool's control words (arrival counts of split pairs)
  int64_t page_bytes;   // bytes between pages
  int64_t q_sb, q_sh, q_st;  // query strides, bytes
  int64_t o_sb, o_sh, o_st;  // output strides, bytes
  const char* q;
  char* out;
  float* part;          // records of record_floats(rows, head_dim), indexed range + pair
  FastDiv page_div;
  int32_t row_bytes;    // bytes between positions of a page
  int32_t head_bytes;   // bytes of one head's run (head_dim elements)
  int32_t num_pages;
  int32_t max_blocks;
  int32_t page_size;
  int32_t kv_heads;
  int32_t group;
  int32_t tokens;
  int32_t rows;
  int32_t batch;
  int32_t max_seq;      // rows are read up to this length (longer ones are flagged)
  int32_t range_chunks; // chunks per range (0: total / waves, at least kMinRangeChunks)
  int32_t waves;        // the launch's waves (one per resident slot)
  float scale_log2;     // softmax scale * log2(e)
  // fp8 cold store (quantised pools; page_size a multiple of 16): a table entry -2 - c names
  // cold page c, whose codes and scales replace the page's K and V.
  const uint8_t* kcodes;
  const uint8_t* vcodes;
  const uint8_t* kscales;
  const uint8_t* vscales;
  int32_t num_cold;
};

// A piece's partial: rows x head_dim unnormalised sums, then the rows' running maxima and sums,
// padded to whole 16-byte vectors.
__host__ __device__ constexpr int64_t record_floats(int64_t rows, int64_t head_dim) {
  return rows * head_dim + (2 * rows + 3) / 4 * 4;
}

template <int E>
__device__ __forceinline__ f32x4 mfma_qk(const u32x4 a, const u32x4 b, f32x4 c) {
  if constexpr (E == kBF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
}

// The 8 elements of a 16-byte vector as fp32 (exact for both 2-byte types).
template <int E>
__device__ __forceinline__ void widen8(const u32x4 w, float (&f)[8]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (E == kBF16) {
      f[2 * i] = __uint_as_float(w[i] << 16);
      f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    } else {
      f[2 * i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] & 0xffffu));
      f[2 * i + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[i] >> 16));
    }
  }
}

template <int E>
__device__ __forceinline__ uint16_t narrow(float f) {
  if constexpr (E == kBF16) {
    // round to nearest even; NaN stays a quiet NaN
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  } else {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// DPP lane moves within each 16-lane row (quad_perm [1,0,3,2], [2,3,0,1], half-row mirror,
// row mirror): four steps combine all 16 lanes of a row.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x141>(v));
  return fmaxf(v, dpp<0x140>(v));
}
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<0xB1>(v);
  v += dpp<0x4E>(v);
  v += dpp<0x141>(v);
  return v + dpp<0x140>(v);
}
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// V rows: each load reads whole 128-byte lines (four positions x 256 bytes), read once.
__device__ __forceinline__ u32x4 ld_page(const char* p) {
  return __builtin_nontemporal_load((const u32x4*)p);
}
// K rows: one load reads 64 bytes of each of 16 positions (half a line), the next load the other
// half; a plain load keeps the line in L1 for it, a nontemporal one fetched it twice (C2 decode
// attention -5 % at 650 positions, -8 % at 1024).
__device__ __forceinline__ u32x4 ld_page_k(const char* p) { return *(const u32x4*)p; }

template <typename OutT, int E>
__device__ __forceinline__ void store_out4(char* p, const f32x4 v) {
  if constexpr (sizeof(OutT) == 4) {
    *(f32x4*)p = v;
  } else {
    uint2 w;
    w.x = (uint32_t)narrow<E>(v[0]) | ((uint32_t)narrow<E>(v[1]) << 16);
    w.y = (uint32_t)narrow<E>(v[2]) | ((uint32_t)narrow<E>(v[3]) << 16);
    *(uint2*)p = w;
  }
}

__device__ __forceinline__ char* out_row(const AttnArgs& a, int b, int kvh, int row) {
  const int hl = row / a.tokens;
  const int i = row - hl * a.tokens;
  return a.out + (int64_t)b * a.o_sb + (int64_t)(kvh * a.group + hl) * a.o_sh + (int64_t)i * a.o_st;
}

// The schedule, computed identically by both kernels from seq_lens: s_len[b] = row b's length
// (clamped to max_seq; longer rows are flagged once), s_incl[b] = chunks of rows 0..b times
// kv_heads.  Run by one wave; returns the total number of chunks.
__device__ int scan_rows(const AttnArgs& a, int lane, int* s_len, int* s_incl, bool report) {
  int base = 0;
  for (int g0 = 0; g0 < a.batch; g0 += kWave) {
    const int b = g0 + lane;
    int len = 0;
    if (b < a.batch) {
      len = a.seq_lens[b];
      if (len > a.max_seq) {
        if (report) atomicOr(a.errors, BARQ_KV_ERRBIT_ATTN_SHORT);
        len = a.max_seq;
      }
      len = len < 0 ? 0 : len;
    }
    int v = (len + kBlock - 1) / kBlock * a.kv_heads;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      const int u = __shfl_up(v, o, kWave);
      if (lane >= o) v += u;
    }
    if (b < a.batch) {
      s_len[b] = len;
      s_incl[b] = base + v;
    }
    base += __shfl(v, kWave - 1, kWave);
  }
  return base;
}

__device__ __forceinline__ int range_chunks(const AttnArgs& a, int total) {
  if (a.range_chunks > 0) return a.range_chunks;
  return max(kMinRangeChunks, (total + a.waves - 1) / a.waves);
}

// Ranges of the flat schedule: [0, na) of pa chunks each, then ranges of pb.  The automatic
// split at two waves per SIMD (up to 8 query rows) gives the first half of the launch's waves --
// each SIMD's first, whose loads are served first -- pa = per + per / 16 chunks and the second
// half pb = per - per / 16, once ranges hold 16 chunks or more (at C2 the second wave on a SIMD
// got its first chunk ~1.4 us later and streamed ~9 % slower).  Otherwise every range holds per.
struct RangeMap {
  int pa, pb, na;
  __device__ int start(int r) const { return r < na ? r * pa : na * pa + (r - na) * pb; }
  __device__ int of(int c) const {
    const int split = na * pa;
    return c < split ? c / pa : na + (c - split) / pb;
  }
};
__device__ __forceinline__ RangeMap range_map(const AttnArgs& a, int total) {
  const int per = range_chunks(a, total);
  RangeMap m{per, per, 0};
  if (a.range_chunks == 0 && a.rows <= 8 && per >= 16) {
    m.pa = per + per / 16;
    m.pb = per - per / 16;
    m.na = a.waves / 2;
  }
  return m;
}

// The row holding chunk c: the first b with s_incl[b] > c (c < total).
__device__ __forceinline__ int find_row(const int* s_incl, int batch, int c) {
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (s_incl[mid] > c) hi = mid; else lo = mid + 1;
  }
  return lo;
}

// Page of block blk0 + idx from the lanes' table window: idx uniform (a scalar) ...
__device__ __forceinline__ int table_scalar(const int (&pt)[kTableRegs], int idx) {
  int page = __builtin_amdgcn_readlane(pt[0], idx & 63);
#pragma unroll
  for (int k = 1; k < kTableRegs; ++k)
    if ((idx >> 6) == k) page = __builtin_amdgcn_readlane(pt[k], idx & 63);
  return page;
}
// ... or per lane (every lane active).
__device__ __forceinline__ int table_lane(const int (&pt)[kTableRegs], int idx) {
  int page = 0;
#pragma unroll
  for (int k = 0; k < kTableRegs; ++k) {
    const int v = __builtin_amdgcn_ds_bpermute((idx & 63) << 2, pt[k]);
    page = (idx >> 6) == k ? v : page;
  }
  return page;
}

// Block-table window of row b: lane j of pt[k] holds block blk0 + 64k + j, for the blocks
// [blk0, blk_end) the piece reads.  issue_table starts the loads; check_table, where the entries
// are first needed, records an entry that names no page of the pool and reads it as page 0, so
// no access leaves the pool.
__device__ __forceinline__ void issue_table(const AttnArgs& a, int b, int blk0, int blk_end, int lane,
                                            int (&pt)[kTableRegs]) {
  const int n = min(kTableEntries, min(blk_end, a.max_blocks) - blk0);
  const int32_t* row = a.block_table + (int64_t)b * a.max_blocks + blk0 + lane;
#pragma unroll
  for (int k = 0; k < kTableRegs; ++k) pt[k] = 64 * k + lane < n ? row[64 * k] : 0;
}
template <bool COLD>
__device__ __forceinline__ void check_table(const AttnArgs& a, int (&pt)[kTableRegs]) {
  bool bad = false;
#pragma unroll
  for (int k = 0; k < kTableRegs; ++k) {
    const int page = pt[k];
    const bool cold_ok = COLD && page <= -2 && -2 - page < a.num_cold;
    const bool bad_k = (uint32_t)page >= (uint32_t)a.num_pages && !cold_ok;
    pt[k] = bad_k ? 0 : page;
    bad |= bad_k;
  }
  if (bad) atomicOr(a.errors, BARQ_KV_ERRBIT_BAD_INDEX);
}
template <bool COLD>
__device__ __forceinline__ void load_table(const AttnArgs& a, int b, int blk0, int blk_end, int lane,
                                           int (&pt)[kTableRegs]) {
  issue_table(a, b, blk0, blk_end, lane, pt);
  check_table<COLD>(a, pt);
}

// Query rows of (row b, kv head kvh) in the A layout of the score MFMA, in the kernel's K order:
// lane (row n16, k-group g) holds, for step st, 8 dims of query row n16 (zero for padding rows) --
// dims 32 st + 8 g (two-byte pages), or 8 kSteps g + 8 st with QUANT (quantised pools: each lane's
// K codes and scales of a position are then one contiguous run, loaded 16 bytes at a time).  Any
// assignment of dims to (step, g) gives the same dot products as long as Q and K share it.
template <int HD, bool QUANT>
__device__ __forceinline__ void issue_query(const AttnArgs& a, int b, int kvh, int lane,
                                            u32x4 (&qv)[Head<HD>::kSteps]) {
  constexpr int kSteps = Head<HD>::kSteps;
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const bool qrow = n16 < a.rows;
  const char* qp = a.q + (int64_t)b * a.q_sb + (int64_t)(kvh * a.group + n16 / a.tokens) * a.q_sh +
                   (int64_t)(n16 % a.tokens) * a.q_st + (QUANT ? 16 * kSteps * g : 16 * g);
#pragma unroll
  for (int st = 0; st < kSteps; ++st)
    qv[st] = qrow ? *(const u32x4*)(qp + (QUANT ? 16 : 64) * st) : u32x4{0, 0, 0, 0};
}

// A piece's first round trip, started by its caller before the row's length is known: the
// block-table window from block 0 (entries the caller's bound allows) and the query rows.
template <int HD>
struct PieceStart {
  int pt[kTableRegs];
  u32x4 qv[Head<HD>::kSteps];
  int blk0;  // the window's first block
};

// K and V of one 16-position chunk for this lane.  K: lane (g, n16) holds dims 32 * step + 8 * g
// .. +7 of position tc + n16 (quantised pools: dims 8 kSteps g + 8 step .. +7, see issue_query);
// V: lane (vpos, vdim) = (lane / (HD / 8), lane % (HD / 8)) holds dims 8 * vdim .. +7 of position
// tc + kVPos * s + vpos.  Positions >= end load nothing and read as zero.
template <int HD, bool UNIFORM, bool PRED, bool COLD>
__device__ __forceinline__ void load_chunk(const AttnArgs& a, const int (&pt)[kTableRegs], int blk0,
                                           const char* kbase, const char* vbase, int tc, int end,
                                           int klane, int vlane, int n16, int g, int vpos, int vdim, int kvh,
                                           u32x4 (&kv)[Head<HD>::kSteps], u32x4 (&vv)[Head<HD>::kVLoads],
                                           bool& cold) {
  constexpr int kSteps = Head<HD>::kSteps;
  constexpr int kVPos = Head<HD>::kVPos;
  constexpr int kVLoads = Head<HD>::kVLoads;
  static_assert(UNIFORM || !COLD, "quantised pools read whole-chunk pages (their K order assumes it)");
  cold = false;
  if constexpr (UNIFORM) {
    // page_size is a multiple of 16: the chunk lies in one page, its base a scalar.
    const uint32_t blk = a.page_div.div((uint32_t)tc);
    const int page = table_scalar(pt, (int)blk - blk0);
    if constexpr (COLD) {
      if (page < 0) {
        // Quantised page: raw codes and scales into the chunk registers, decoded just before the
        // chunk is computed (so the loads stay in flight meanwhile).  K: lane (g, n16) takes 8
        // codes of dims 32 st + 8 g of position tc + n16, and their 8 per-channel scales; V: 8
        // codes of dims 8 vdim of position tc + kVPos s + vpos, and that position's scale.
        cold = true;
        const int c = -2 - page;
        const int t0 = tc - (int)(blk * (uint32_t)a.page_size);
        const int64_t head = (int64_t)kvh * HD;
        const int64_t code_page = (int64_t)c * a.page_size * a.kv_heads * HD;
        // (the quantised kernels' K layout: lane g's codes and scales for every step are one run
        // of 8 kSteps bytes, loaded 16 bytes at a time)
        const uint8_t* kc =
            a.kcodes + code_page + (int64_t)(t0 + n16) * a.kv_heads * HD + head + 8 * kSteps * g;
        const uint8_t* ks = a.kscales + ((int64_t)c * a.kv_heads) * HD + head + 8 * kSteps * g;
        const bool in = !PRED || tc + n16 < end;
#pragma unroll
        for (int st = 0; st < kSteps; st += 2) {
          const u32x4 cw = in ? *(const u32x4*)(kc + 8 * st) : u32x4{0, 0, 0, 0};
          const u32x4 sw = *(const u32x4*)(ks + 8 * st);
          kv[st] = u32x4{cw[0], cw[1], sw[0], sw[1]};
          kv[st + 1] = u32x4{cw[2], cw[3], sw[2], sw[3]};
        }
#pragma unroll
        for (int s = 0; s < kVLoads; ++s) {
          const int t = t0 + kVPos * s + vpos;
          const bool in = !PRED || tc + kVPos * s + vpos < end;
          const uint2 cw = in ? *(const uint2*)(a.vcodes + code_page + (int64_t)t * a.kv_heads * HD + head + 8 * vdim)
                              : uint2{0, 0};
          const uint32_t sv = in ? a.vscales[((int64_t)c * a.page_size + t) * a.kv_heads + kvh] : 127u;
          vv[s] = u32x4{cw.x, cw.y, sv, 0};
        }
        return;
      }
    }
    const int64_t base = (int64_t)page * a.page_bytes +
                         (int64_t)(tc - (int)(blk * (uint32_t)a.page_size)) * a.row_bytes;
    const char* kp = kbase + base + klane;
    const char* vp = vbase + base + vlane;
#pragma unroll
    for (int st = 0; st < kSteps; ++st)
      kv[st] = (!PRED || tc + n16 < end) ? ld_page_k(kp + (COLD ? 16 : 64) * st) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kVLoads; ++s)
      vv[s] = (!PRED || tc + kVPos * s + vpos < end) ? ld_page(vp + kVPos * s * a.row_bytes) : u32x4{0, 0, 0, 0};
  } else {
    const int tk = min(tc + n16, end - 1);
    const uint32_t bk = a.page_div.div((uint32_t)tk);
    const int pk = table_lane(pt, (int)bk - blk0);
    const char* kp = kbase + (int64_t)pk * a.page_bytes +
                     (int64_t)(tk - (int)(bk * (uint32_t)a.page_size)) * a.row_bytes + 16 * g;
#pragma unroll
    for (int st = 0; st < kSteps; ++st)
      kv[st] = (!PRED || tc + n16 < end) ? ld_page_k(kp + 64 * st) : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < kVLoads; ++s) {
      const int tv = min(tc + kVPos * s + vpos, end - 1);
      const uint32_t bv = a.page_div.div((uint32_t)tv);
      const int pv = table_lane(pt, (int)bv - blk0);
      const char* vp = vbase + (int64_t)pv * a.page_bytes +
                       (int64_t)(tv - (int)(bv * (uint32_t)a.page_size)) * a.row_bytes + 16 * vdim;
      vv[s] = (!PRED || tc + kVPos * s + vpos < end) ? ld_page(vp) : u32x4{0, 0, 0, 0};
    }
  }
}

// A chunk of a two-byte pool with whole-chunk pages whose positions past `end` read position
// end - 1 (the causal mask gives them probability 0): every lane loads, no branch around the loads.
// QORDER: K in the quantised pools' order (issue_query), for the two-byte pages of such a pool.
template <int HD, bool QORDER = false>
__device__ __forceinline__ void load_chunk_clamped(const AttnArgs& a, const int (&pt)[kTableRegs], int blk0,
                                                   const char* kbase, const char* vbase, int tc, int end, int n16,
                                                   int g, int vpos, int vdim, u32x4 (&kv)[Head<HD>::kSteps],
                                                   u32x4 (&vv)[Head<HD>::kVLoads]) {
  constexpr int kSteps = Head<HD>::kSteps;
  constexpr int kVPos = Head<HD>::kVPos;
  constexpr int kVLoads = Head<HD>::kVLoads;
  const uint32_t blk = a.page_div.div((uint32_t)tc);
  // (QORDER: a quantised block here, -2 - c, breaks the pool's order -- its caller reports it --
  // and reads page 0 instead of memory before the pages)
  const int page = QORDER ? max(table_scalar(pt, (int)blk - blk0), 0) : table_scalar(pt, (int)blk - blk0);
  const int64_t base =
      (int64_t)page * a.page_bytes + (int64_t)(tc - (int)(blk * (uint32_t)a.page_size)) * a.row_bytes;
  const int lastp = end - 1 - tc;  // >= 15 for a whole chunk
  const char* kp = kbase + base + min(n16, lastp) * a.row_bytes + (QORDER ? 16 * kSteps * g : 16 * g);
#pragma unroll
  for (int st = 0; st < kSteps; ++st) kv[st] = ld_page_k(kp + (QORDER ? 16 : 64) * st);
#pragma unroll
  for (int s = 0; s < kVLoads; ++s)
    vv[s] = ld_page(vbase + base + min(kVPos * s + vpos, lastp) * a.row_bytes + 16 * vdim);
}

// A quantised chunk (its block's table entry is -2 - c, c its quantised block), positions past
// `end` reading position end - 1 as load_chunk_clamped does: every lane loads, no branch around
// the loads.  K as load_chunk lays it out; V: the 8 codes of each of the lane's positions, and
// one scale byte a lane, position lane % 16's (spread to the lanes at the chunk's products).
template <int HD>
__device__ __forceinline__ void load_cold_clamped(const AttnArgs& a, const int (&pt)[kTableRegs], int blk0, int tc,
                                                  int end, int n16, int g, int vpos, int vdim, int kvh,
                                                  u32x4 (&kv)[Head<HD>::kSteps], uint2 (&vc)[Head<HD>::kVLoads],
                                                  uint32_t& vs) {
  constexpr int kSteps = Head<HD>::kSteps;
  constexpr int kVPos = Head<HD>::kVPos;
  constexpr int kVLoads = Head<HD>::kVLoads;
  const uint32_t blk = a.page_div.div((uint32_t)tc);
  const int c = -2 - table_scalar(pt, (int)blk - blk0);
  const int t0 = tc - (int)(blk * (uint32_t)a.page_size);
  const int lastp = end - 1 - tc;
  const int64_t head = (int64_t)kvh * HD;
  const int64_t code_page = (int64_t)c * a.page_size * a.kv_heads * HD;
  const uint8_t* kc = a.kcodes + code_page + (int64_t)(t0 + min(n16, lastp)) * a.kv_heads * HD + head + 8 * kSteps * g;
  const uint8_t* ks = a.kscales + ((int64_t)c * a.kv_heads) * HD + head + 8 * kSteps * g;
#pragma unroll
  for (int st = 0; st < kSteps; st += 2) {
    const u32x4 cw = *(const u32x4*)(kc + 8 * st);
    const u32x4 sw = *(const u32x4*)(ks + 8 * st);
    kv[st] = u32x4{cw[0], cw[1], sw[0], sw[1]};
    kv[st + 1] = u32x4{cw[2], cw[3], sw[2], sw[3]};
  }
#pragma unroll
  for (int s = 0; s < kVLoads; ++s) {
    const int t = t0 + min(kVPos * s + vpos, lastp);
    vc[s] = *(const uint2*)(a.vcodes + code_page + (int64_t)t * a.kv_heads * HD + head + 8 * vdim);
  }
  vs = a.vscales[((int64_t)c * a.page_size + t0 + min(n16, lastp)) * a.kv_heads + kvh];
}

// One register of a quantised chunk (8 codes and their scale bytes: K's per channel, V's -- value
// -- the position's one) -> 8 two-byte values: exponent arithmetic where it applies, else the
// exact element path.
template <int E>
__device__ __forceinline__ u32x4 dequant_vector(const u32x4 x, bool value) {
  const uint32_t s0 = value ? x[2] * 0x01010101u : x[2];
  const uint32_t s1 = value ? s0 : x[3];
  uint32_t o[4];
  if (barq_fp8::dequant8_fast_ok<E>(x[0], x[1], s0, s1)) {
    barq_fp8::dequant8_fast<E>(x[0], x[1], s0, s1, o);
  } else {
    o[0] = barq_fp8::dequant2_inline<E>(x[0], s0);
    o[1] = barq_fp8::dequant2_inline<E>(x[0] >> 16, s0 >> 16);
    o[2] = barq_fp8::dequant2_inline<E>(x[1], s1);
    o[3] = barq_fp8::dequant2_inline<E>(x[1] >> 16, s1 >> 16);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

// A quantised chunk's K (VALUE false: codes and per-channel scales per register) or V (VALUE
// true: codes and the position's scale) -> two-byte values.  When every vector of every lane
// qualifies, exponent arithmetic decodes the registers unrolled; otherwise (a zero, subnormal or
// NaN code, or an extreme scale somewhere in the wave) one out-of-line function takes the
// registers by value and returns them decoded, so the rare path adds no register pressure to the
// common one (inlined, even as a rolled loop, it made the quantised chunk loops spill).
template <int N>
struct ChunkRegs {
  u32x4 r[N];
};
template <int E, bool VALUE, int N>
__device__ __noinline__ ChunkRegs<N> dequant_regs_exact(ChunkRegs<N> x) {
#pragma unroll
  for (int n = 0; n < N; ++n) x.r[n] = dequant_vector<E>(x.r[n], VALUE);
  return x;
}

template <int E, bool VALUE, int N>
__device__ __forceinline__ void dequant_regs(u32x4 (&r)[N]) {
  bool fast = true;
#pragma unroll
  for (int n = 0; n < N; ++n) {
    const uint32_t s0 = VALUE ? r[n][2] * 0x01010101u : r[n][2];
    const uint32_t s1 = VALUE ? r[n][2] * 0x01010101u : r[n][3];
    fast = fast && barq_fp8::dequant8_fast_ok<E>(r[n][0], r[n][1], s0, s1);
  }
  if (__builtin_amdgcn_ballot_w64(!fast) == 0) {
#pragma unroll
    for (int n = 0; n < N; ++n) {
      const uint32_t s0 = VALUE ? r[n][2] * 0x01010101u : r[n][2];
      const uint32_t s1 = VALUE ? r[n][2] * 0x01010101u : r[n][3];
      uint32_t o[4];
      barq_fp8::dequant8_fast<E>(r[n][0], r[n][1], s0, s1, o);
      r[n] = u32x4{o[0], o[1], o[2], o[3]};
    }
    return;
  }
  ChunkRegs<N> x;
#pragma unroll
  for (int n = 0; n < N; ++n) x.r[n] = r[n];
  x = dequant_regs_exact<E, VALUE, N>(x);
#pragma unroll
  for (int n = 0; n < N; ++n) r[n] = x.r[n];
}

// Fast operands from a quantised chunk (scale bytes in [64, 191], checked per chunk): the codes
// are converted by the hardware (gfx950 decodes OCP E4M3 exactly, zero and subnormal codes
// included) and multiplied by 2^(s - 127) -- exact in fp32 -- then rounded to the two-byte type
// as the dequantising gather rounds them (bf16: exact, the top half; fp16: nearest even), so K's
// operand holds exactly the dequantised value.  V needs no scale here: its per-position scale
// multiplies the probability (exact: a power of two).  A NaN code reads as NaN either way, and
// the hardware's +0 for code 0x80 (-0) changes no product or sum.
// Every scale byte of a chunk's K registers (VALUE false: 8 per register) or V registers (the
// position's byte) in 64..191: its top two bits are 01 or 10.  K is checked before the scores and
// V before P.V, so neither waits for the other's loads.
template <bool VALUE, int N>
__device__ __forceinline__ bool scales_moderate(const u32x4 (&r)[N]) {
  uint32_t ok = 0x40404040u;
#pragma unroll
  for (int n = 0; n < N; ++n)
    ok &= VALUE ? (((r[n][2] >> 1) ^ r[n][2]) | 0x40404000u) : (((r[n][2] >> 1) ^ r[n][2]) & ((r[n][3] >> 1) ^ r[n][3]));
  return (ok & 0x40404040u) == 0x40404040u;
}

__device__ __forceinline__ float e8m0_float(uint32_t s) { return __uint_as_float(s << 23); }

template <int E>
__device__ __forceinline__ u32x4 k_operand(const u32x4 x) {
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t w = x[j], sw = x[2 + j];
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    const float f0 = lo[0] * e8m0_float(sw & 0xFFu), f1 = lo[1] * e8m0_float((sw >> 8) & 0xFFu);
    const float f2 = hi[0] * e8m0_float((sw >> 16) & 0xFFu), f3 = hi[1] * e8m0_float(sw >> 24);
    if constexpr (E == kBF16) {
      o[2 * j] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
      o[2 * j + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
    } else {  // round to nearest even, as the dequantised values are (fp16's range is narrow)
      o[2 * j] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f0) |
                 ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f1) << 16);
      o[2 * j + 1] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f2) |
                     ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f3) << 16);
    }
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

__device__ __forceinline__ void v_operand(const u32x4 x, float (&f)[8]) {
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[j], false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[j], true);
    f[4 * j] = lo[0];
    f[4 * j + 1] = lo[1];
    f[4 * j + 2] = hi[0];
    f[4 * j + 3] = hi[1];
  }
}

template <int HD, int E, int R, bool UNIFORM, typename OutT, bool COLD, bool PRE = false>
__device__ void attend_piece(const AttnArgs& a, float (&lp)[kBlock][kMaxRows],
                             u32x4 (&lq)[Head<HD>::kSteps][kWave], int b, int kvh, int len, int t_begin,
                             int t_end, bool whole, float* pr, const PieceStart<HD>* pre = nullptr) {
  constexpr int kSteps = Head<HD>::kSteps;
  constexpr int kVLanes = Head<HD>::kVLanes;
  constexpr int kVPos = Head<HD>::kVPos;
  constexpr int kVLoads = Head<HD>::kVLoads;
  const int lane = threadIdx.x & (kWave - 1);
  const int n16 = lane & 15;
  const int g = lane >> 4;
  const int vpos = lane / kVLanes;  // V: position slot and 8-dim group of this lane
  const int vdim = lane % kVLanes;
  const int M = a.rows;
  const int T = a.tokens;

  // The block-table window and the query rows load together: one round trip before the first
  // chunk's loads (PRE: the caller started both, the window from block pre->blk0, mostly before
  // it knew the row's length; entries past the piece's blocks are dropped unchecked).  The query rows are
  // kept in LDS.
  int blk0 = PRE ? pre->blk0 : (int)a.page_div.div((uint32_t)t_begin);
  const int blk_end = t_end > t_begin ? (int)a.page_div.div((uint32_t)(t_end - 1)) + 1 : blk0;
  int pt[kTableRegs];
  // The pair kernel keeps its query fragments in registers (it has them to spare), the others
  // read them from LDS for every chunk.
  constexpr bool kQReg = PRE && !COLD && R == 1;
  u32x4 qreg[kSteps];
  {
    u32x4 qv[kSteps];
    if constexpr (PRE) {
#pragma unroll
      for (int k = 0; k < kTableRegs; ++k) pt[k] = 64 * k + lane < blk_end - blk0 ? pre->pt[k] : 0;
#pragma unroll
      for (int st = 0; st < kSteps; ++st) qv[st] = pre->qv[st];
    } else {
      issue_table(a, b, blk0, blk_end, lane, pt);
      issue_query<HD, COLD>(a, b, kvh, lane, qv);
    }
#pragma unroll
    for (int st = 0; st < kSteps; ++st) {
      if constexpr (kQReg)
        qreg[st] = qv[st];
      else
        lq[st][lane] = qv[st];
    }
  }
  check_table<COLD>(a, pt);

  const char* kbase = a.kpages + (int64_t)kvh * a.head_bytes;
  const char* vbase = a.vpages + (int64_t)kvh * a.head_bytes;
  const int klane = n16 * a.row_bytes + (COLD ? 16 * kSteps * g : 16 * g);  // the K layout (issue_query)
  const int vlane = vpos * a.row_bytes + 16 * vdim;

  float m_run[4], l_part[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = -INFINITY;
    l_part[r] = 0.f;
  }
  f32x4 acc[R][8];
#pragma unroll
  for (int r2 = 0; r2 < R; ++r2)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r2][e] = f32x4{0.f, 0.f, 0.f, 0.f};

  // Slide the table window when the chunk's last block leaves it (every 254+ blocks).
  auto slide = [&](int tc) {
    const int last = (int)a.page_div.div((uint32_t)min(tc + kBlock, t_end) - 1u);
    if (last - blk0 >= kTableEntries) {
      blk0 = (int)a.page_div.div((uint32_t)tc);
      load_table<COLD>(a, b, blk0, blk_end, lane, pt);
    }
  };
  // A chunk of the piece, whole or its partial last one (lanes past t_end load nothing).
  auto load_any = [&](int tc, u32x4 (&kv)[kSteps], u32x4 (&vv)[kVLoads], bool& cold) {
    slide(tc);
    if (tc + kBlock <= t_end)
      load_chunk<HD, UNIFORM, false, COLD>(a, pt, blk0, kbase, vbase, tc, t_end, klane, vlane, n16, g, vpos, vdim,
                                           kvh, kv, vv, cold);
    else
      load_chunk<HD, UNIFORM, true, COLD>(a, pt, blk0, kbase, vbase, tc, t_end, klane, vlane, n16, g, vpos, vdim,
                                          kvh, kv, vv, cold);
  };

  // codes: the chunk registers hold a quantised chunk with moderate scales (see k_operand).
  // kcodes: the K registers hold a quantised chunk's codes with moderate scales (k_operand);
  // vcold: the V registers hold a quantised chunk's codes, checked here before P.V.
  // (with the rescale under a branch, the quantised flat kernel and 8+ rows on the flat schedule
  // or over quantised pages spill)
  constexpr bool kLazyMax = R == 1 ? !COLD || PRE : R == 2 && PRE && !COLD;
  auto compute = [&](int tc, const u32x4 (&kv)[kSteps], u32x4 (&vv)[kVLoads], bool kcodes, bool vcold) {
    // Scores: lane (g, n16), register r = row 4g + r, position tc + n16; log2 units.
    f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < kSteps; ++st)
      sc = mfma_qk<E>(kQReg ? qreg[st] : lq[st][lane], (COLD && kcodes) ? k_operand<E>(kv[st]) : kv[st], sc);
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) x[r] = sc[r] * a.scale_log2;
    // Every position of the chunk visible to every row?  Else mask (position > len - T + i).
    if (tc + kBlock + T - 1 > len) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 4 * g + r;
        if (tc + n16 > len - T + row % T) x[r] = -INFINITY;
      }
    }
    if constexpr (kLazyMax) {
      // The running maximum moves only when a score of the chunk exceeds it by more than 8
      // (log2 units), so most chunks skip the row reductions and the rescale.  Probabilities are then at most 2^8 against the row's reference maximum
      // (sums stay far from the float range; the output is the same quotient, rounded apart).
      bool up = false;
#pragma unroll
      for (int r = 0; r < 4; ++r) up = up || x[r] > m_run[r] + 8.0f;
      if (__builtin_amdgcn_ballot_w64(up && g < R) != 0) {
        float alpha[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float mnew = fmaxf(m_run[r], row16_max(x[r]));
          const float mu = mnew == -INFINITY ? 0.f : mnew;
          alpha[r] = __builtin_amdgcn_exp2f(m_run[r] - mu);
          l_part[r] *= alpha[r];
          m_run[r] = mnew;
        }
#pragma unroll
        for (int r2 = 0; r2 < R; ++r2)
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const float al = lane_value(alpha[m], 16 * r2);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[r2][e][m] *= al;
          }
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float mu = m_run[r] == -INFINITY ? 0.f : m_run[r];
        x[r] = __builtin_amdgcn_exp2f(x[r] - mu);
        l_part[r] += x[r];
      }
      if (g < R) *(f32x4*)&lp[n16][4 * g] = f32x4{x[0], x[1], x[2], x[3]};
    } else {
      float alpha[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float mnew = fmaxf(m_run[r], row16_max(x[r]));
        const float mu = mnew == -INFINITY ? 0.f : mnew;
        alpha[r] = __builtin_amdgcn_exp2f(m_run[r] - mu);
        x[r] = __builtin_amdgcn_exp2f(x[r] - mu);
        l_part[r] = l_part[r] * alpha[r] + x[r];
        m_run[r] = mnew;
      }
      if (g < R) *(f32x4*)&lp[n16][4 * g] = f32x4{x[0], x[1], x[2], x[3]};
      // Every chunk rescales every row's accumulators (alpha is exactly 1 where a row's maximum
      // did not move): with the multiply under a branch the compiler kept two copies of the
      // accumulators live at 8 and 16 query rows (spills).
#pragma unroll
      for (int r2 = 0; r2 < R; ++r2)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const float al = lane_value(alpha[m], 16 * r2);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[r2][e][m] *= al;
        }
    }
    bool vcodes = false;
    if (COLD && vcold) {
      vcodes = __builtin_amdgcn_ballot_w64(!scales_moderate<true>(vv)) == 0;
      if (!vcodes) dequant_regs<E, true>(vv);
    }
    // P.V: lane 4b' + n of the 4x4x1 MFMA block b' takes position kVPos * s + vpos of the chunk
    // (the four lanes of a block share it) and dims 8 * vdim + e.
#pragma unroll
    for (int s = 0; s < kVLoads; ++s) {
      float vf[8];
      float vs = 1.0f;  // a quantised position's scale, moved onto its probability
      if (COLD && vcodes) {
        v_operand(vv[s], vf);
        vs = e8m0_float(vv[s][2]);
      } else {
        widen8<E>(vv[s], vf);
      }
#pragma unroll
      for (int r2 = 0; r2 < R; ++r2) {
        const float pa = lp[kVPos * s + vpos][4 * r2 + (lane & 3)] * vs;
#pragma unroll
        for (int e = 0; e < 8; ++e)
          acc[r2][e] = __builtin_amdgcn_mfma_f32_4x4x1f32(pa, vf[e], acc[r2][e], 0, 0, 0);
      }
    }
  };

  // Two register buffers: the next chunk's loads are in flight while one is computed (a third
  // spills, or for 4 query rows runs slower, with the accumulators in registers).
  u32x4 kr[2][kSteps], vr[2][kVLoads];
  bool cr[2] = {false, false};  // the buffer holds codes and scales (wave-uniform)
  int tc = t_begin;
  auto step = [&](int i) {
    bool kcodes = false;
    if (COLD && cr[i]) {
      kcodes = __builtin_amdgcn_ballot_w64(!scales_moderate<false>(kr[i])) == 0;
      if (!kcodes) dequant_regs<E, false>(kr[i]);
    }
    compute(tc, kr[i], vr[i], kcodes, COLD && cr[i]);
    tc += kBlock;
  };
  if constexpr (PRE && !COLD && R == 1) {
    // Pair kernel, up to 4 query rows, two-byte pages (its table window holds every block of the
    // pair: no slide).  The wait the compiler puts before a chunk's products counts the loads
    // issued after that chunk's; where one path to the products skips the next chunk's loads, or
    // loads it under a lane mask, that count is the smaller one on every path and each chunk also
    // waits for part of the next chunk's data.  So the next chunk, whole or partial, is loaded on
    // every path of the loop, clamped instead of masked, and the loop is left before a load.
    // (The 8+ row variants keep the ring below: this form's registers spill there; quantised
    // pools take the loops that follow.)
    auto load_clamped = [&](int t, u32x4 (&kv)[kSteps], u32x4 (&vv)[kVLoads]) {
      load_chunk_clamped<HD>(a, pt, blk0, kbase, vbase, t, t_end, n16, g, vpos, vdim, kv, vv);
    };
    if (tc < t_end) {
      load_clamped(tc, kr[0], vr[0]);
      for (;;) {
        if (tc + kBlock >= t_end) {
          step(0);
          break;
        }
        load_clamped(tc + kBlock, kr[1], vr[1]);
        __builtin_amdgcn_sched_barrier(0);
        step(0);
        if (tc + kBlock >= t_end) {
          step(1);
          break;
        }
        load_clamped(tc + kBlock, kr[0], vr[0]);
        __builtin_amdgcn_sched_barrier(0);
        step(1);
      }
    }
  } else if constexpr (PRE && COLD && R == 1) {
    // The same loop over a quantised pool: its quantised blocks lead every row, so the piece is a
    // run of quantised chunks, then one of two-byte chunks (the residual window), each loop
    // loading every chunk whole and clamped.  (One loop over both kinds, a branch choosing each
    // chunk's loads, waits for every load in flight before each chunk's products.)
    auto cold_at = [&](int t) { return table_scalar(pt, (int)a.page_div.div((uint32_t)t) - blk0) < 0; };
    u32x4 ck[2][kSteps];
    uint2 cvc[2][kVLoads];
    uint32_t cvs[2];
    auto load_cold = [&](int t, u32x4 (&kv)[kSteps], uint2 (&vc)[kVLoads], uint32_t& vs) {
      load_cold_clamped<HD>(a, pt, blk0, t, t_end, n16, g, vpos, vdim, kvh, kv, vc, vs);
    };
    bool misordered = false;  // a quantised block after a two-byte one (never made by the pool)
    auto load_hot = [&](int t, u32x4 (&kv)[kSteps], u32x4 (&vv)[kVLoads]) {
      misordered |= cold_at(t);
      load_chunk_clamped<HD, true>(a, pt, blk0, kbase, vbase, t, t_end, n16, g, vpos, vdim, kv, vv);
    };
    auto step_cold = [&](u32x4 (&kv)[kSteps], const uint2 (&vc)[kVLoads], uint32_t vs) {
      const bool kcodes = __builtin_amdgcn_ballot_w64(!scales_moderate<false>(kv)) == 0;
      if (!kcodes) dequant_regs<E, false>(kv);
      u32x4 vv[kVLoads];  // codes and the position's scale, as load_chunk lays a quantised V out
#pragma unroll
      for (int s = 0; s < kVLoads; ++s) vv[s] = u32x4{vc[s].x, vc[s].y, (uint32_t)__shfl((int)vs, kVPos * s + vpos), 0};
      compute(tc, kv, vv, kcodes, true);
      tc += kBlock;
    };
    auto step_hot = [&](int i) {
      compute(tc, kr[i], vr[i], false, false);
      tc += kBlock;
    };
    if (tc < t_end && cold_at(tc)) {
      load_cold(tc, ck[0], cvc[0], cvs[0]);
      for (;;) {
        if (tc + kBlock >= t_end || !cold_at(tc + kBlock)) {
          step_cold(ck[0], cvc[0], cvs[0]);
          break;
        }
        load_cold(tc + kBlock, ck[1], cvc[1], cvs[1]);
        __builtin_amdgcn_sched_barrier(0);
        step_cold(ck[0], cvc[0], cvs[0]);
        if (tc + kBlock >= t_end || !cold_at(tc + kBlock)) {
          step_cold(ck[1], cvc[1], cvs[1]);
          break;
        }
        load_cold(tc + kBlock, ck[0], cvc[0], cvs[0]);
        __builtin_amdgcn_sched_barrier(0);
        step_cold(ck[1], cvc[1], cvs[1]);
      }
    }
    if (tc < t_end) {
      load_hot(tc, kr[0], vr[0]);
      for (;;) {
        if (tc + kBlock >= t_end) {
          step_hot(0);
          break;
        }
        load_hot(tc + kBlock, kr[1], vr[1]);
        __builtin_amdgcn_sched_barrier(0);
        step_hot(0);
        if (tc + kBlock >= t_end) {
          step_hot(1);
          break;
        }
        load_hot(tc + kBlock, kr[0], vr[0]);
        __builtin_amdgcn_sched_barrier(0);
        step_hot(1);
      }
    }
    if (misordered && lane == 0) atomicOr(a.errors, BARQ_KV_ERRBIT_BAD_INDEX);
  } else {
    if (tc < t_end) {
      load_any(tc, kr[0], vr[0], cr[0]);
      for (;;) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          if (tc + kBlock < t_end) load_any(tc + kBlock, kr[1 - i], vr[1 - i], cr[1 - i]);
          __builtin_amdgcn_sched_barrier(0);
          step(i);
          if (tc >= t_end) goto chunks_done;
        }
      }
    }
  chunks_done:;
  }

  // Row sums across the 16 lanes of each row group; P.V partials across the position slots.
#pragma unroll
  for (int r = 0; r < 4; ++r) l_part[r] = row16_sum(l_part[r]);
#pragma unroll
  for (int r2 = 0; r2 < R; ++r2)
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        float v = acc[r2][e][m];
#pragma unroll
        for (int o = kVLanes; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
        acc[r2][e][m] = v;
      }
  // Lanes 0 .. HD / 8 - 1 now hold dims 8 * lane .. +7 of every row; lanes 16g .. 16g+15 hold
  // the maxima and sums of rows 4g .. 4g+3.  A partial goes to the record at pr.
#pragma unroll
  for (int r2 = 0; r2 < R; ++r2)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int row = 4 * r2 + m;
      if (row >= M) break;
      const float mr = lane_value(m_run[m], 16 * r2);
      const float lr = lane_value(l_part[m], 16 * r2);
      if (whole) {
        if (lane < kVLanes) {
          const float inv = lr > 0.f ? 1.f / lr : 0.f;
          char* o = out_row(a, b, kvh, row) + (int64_t)(8 * lane) * sizeof(OutT);
          store_out4<OutT, E>(o, f32x4{acc[r2][0][m], acc[r2][1][m], acc[r2][2][m], acc[r2][3][m]} * inv);
          store_out4<OutT, E>(o + 4 * sizeof(OutT),
                              f32x4{acc[r2][4][m], acc[r2][5][m], acc[r2][6][m], acc[r2][7][m]} * inv);
        }
      } else {
        if (lane < kVLanes) {
          float* dst = pr + (int64_t)row * HD + 8 * lane;
          *(f32x4*)dst = f32x4{acc[r2][0][m], acc[r2][1][m], acc[r2][2][m], acc[r2][3][m]};
          *(f32x4*)(dst + 4) = f32x4{acc[r2][4][m], acc[r2][5][m], acc[r2][6][m], acc[r2][7][m]};
        } else if (lane == kVLanes) {
          pr[(int64_t)M * HD + row] = mr;
          pr[(int64_t)M * HD + M + row] = lr;
        }
      }
    }
}

// One wave per workgroup, one workgroup per resident slot: ranges r = blockIdx.x, + gridDim.x,
// ... of the flat chunk list.  UNIFORM: page_size is a multiple of 16.  R: groups of 4 query
// rows (rows <= 4 * R).  HD: the head size.
template <int HD, int E, int R, bool UNIFORM, typename OutT, bool COLD>
__global__ __launch_bounds__(kWave)
__attribute__((amdgpu_waves_per_eu(R <= 2 && HD <= 128 ? 2 : 1, R <= 2 && HD <= 128 ? 2 : 1)))
void attention_flat_kernel(const AttnArgs a) {
  __shared__ float lp[kBlock][kMaxRows];             // probabilities, staged for the P.V operand layout
  __shared__ u32x4 lq[Head<HD>::kSteps][kWave];      // the piece's query fragments
  __shared__ int s_len[kMaxBatch];
  __shared__ int s_incl[kMaxBatch];

  const int lane = threadIdx.x;
  const int total = scan_rows(a, lane, s_len, s_incl, blockIdx.x == 0 && lane == 0);
  const RangeMap rm = range_map(a, total);
  for (int r = blockIdx.x; rm.start(r) < total; r += gridDim.x) {
    int c = rm.start(r);
    const int c_end = min(total, rm.start(r + 1));
    while (c < c_end) {
      const int b = find_row(s_incl, a.batch, c);
      const int row_first = b > 0 ? s_incl[b - 1] : 0;
      const int len = s_len[b];
      const int nch = (len + kBlock - 1) / kBlock;
      const int kvh = (c - row_first) / nch;
      const int pair_first = row_first + kvh * nch;
      const int k0 = c - pair_first;
      const int piece_end = min(c_end, pair_first + nch);
      const bool whole = k0 == 0 && piece_end == pair_first + nch;
      attend_piece<HD, E, R, UNIFORM, OutT, COLD>(
          a, lp, lq, b, kvh, len, kBlock * k0, min(len, kBlock * (k0 + piece_end - c)), whole,
          a.part + ((int64_t)r + (int64_t)b * a.kv_heads + kvh) * record_floats(a.rows, HD));
      c = piece_end;
    }
  }
}

// Many short pairs (C2: 16 rows x 8 kv heads, ~650 positions): one workgroup of W waves per
// (row, kv head).  Wave w streams nch / W chunks of its pair (one more for the first nch % W
// waves), leaves its partial record in LDS, and the workgroup folds the W records into the
// output (the merge kernel's base-2 online-softmax fold): one launch, each pair's bytes read
// once.  A wave with no chunks leaves a neutral record (maximum -inf, sum 0).
//
// S = 2, or kSplitAny for the grid's count (launches whose S x pairs workgroups are resident at
// once): workgroups p, p + pairs, ... share pair p.  A row is cut over the first k of them, k the
// most that give each at least pair_part_chunks<R>() chunks (ranges dealt to their k x W waves in
// turn), and the others leave at once (k = 1: the first takes the row alone).  A split pair's
// workgroups each fold their waves in LDS, publish the folded record in the workspace and
// arrive on the pair's count in ctrl; the last to arrive folds the k records into the output and
// sets the count back to 0.  No workgroup waits for another, so the grid needs no co-residency
// to finish.  The records are written with agent-scope atomic stores, which write through to
// the device's coherence point (`global_store ... sc1`), every one of them complete
// (s_waitcnt vmcnt(0), then the barrier) before the arrival; the last arrival reads them with
// agent-scope atomic loads (`sc1`) issued after its count returned, every record's loads at
// once.  An agent-scope release fence would write back the whole L2 (~1.7 us); this exchange
// costs ~1.3 us in all.
template <int HD, int E, int R, typename OutT, bool COLD, int W, int S>
__global__ __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(R <= 2 ? 2 : 1, R <= 2 ? 2 : 1)))
void attention_pair_kernel(const AttnArgs a) {
  static_assert(S == 1 || S == 2 || S == kSplitAny || S == kSplitLong,
                "one, two or the grid's count of workgroups a pair");
  constexpr bool kGrid = S == kSplitAny || S == kSplitLong;  // the workgroups a pair: the grid's count
  constexpr int kRecMax = (int)record_floats(4 * R, HD);
  constexpr int kQuads = HD / 4;
  __shared__ float lp[W][kBlock][kMaxRows];
  __shared__ u32x4 lq[W][Head<HD>::kSteps][kWave];
  __shared__ float s_rec[W * kRecMax];
  __shared__ int s_arrived;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / kWave));
  // (The first workgroups of a launch compute this before their first load: a compare where it
  // can be one.)
  const int pairs = kGrid ? a.batch * a.kv_heads : (int)gridDim.x / S;
  const int nsplit = kGrid ? (int)gridDim.x / pairs : S;
  const int half = S == 1   ? 0
                   : S == 2 ? (int)((int)blockIdx.x >= pairs)
                            : (int)blockIdx.x / pairs;  // this workgroup's part of the pair
  const int pair = (int)blockIdx.x - half * pairs;
  const int b = pair / a.kv_heads;
  const int kvh = pair - b * a.kv_heads;
  // The row's length, the table window (every block max_seq allows) and the query rows load
  // together.
  int len = a.seq_lens[b];
  PieceStart<HD> ps;
  ps.blk0 = 0;
  issue_table(a, b, 0, (int)a.page_div.div((uint32_t)a.max_seq + a.page_size - 1), threadIdx.x & (kWave - 1), ps.pt);
  issue_query<HD, COLD>(a, b, kvh, threadIdx.x & (kWave - 1), ps.qv);
  if (len > a.max_seq) {
    if (threadIdx.x == 0 && kvh == 0 && !half) atomicOr(a.errors, BARQ_KV_ERRBIT_ATTN_SHORT);
    len = a.max_seq;
  }
  len = max(len, 0);
  const int nch = (len + kBlock - 1) / kBlock;
  int kparts = S == 1 ? 1 : min(nsplit, max(1, nch / pair_part_chunks<R>()));
  if (S == kSplitLong && kparts > 8) kparts = min(nsplit, max(8, nch / kLongPartChunks));
  const bool split = kparts > 1;
  if (half >= kparts) return;
  // The first waves take the remainder: waves 0 .. 3 are each SIMD's first, whose loads are
  // served first (the second wave on a SIMD gets its first chunk ~1.5 us later).  Rows whose
  // blocks all lie in the prologue's window deal their ranges to the workgroups in turn; longer
  // ones (kSplitLong) give each workgroup a contiguous part, which loads its own window.
  int c0, c1;
  if (S != kSplitLong || (int)a.page_div.div((uint32_t)max(kBlock * nch - 1, 0)) < kTableEntries) {
    const int parts = kparts * W;
    const int gw = w * kparts + half;
    const int base = nch / parts, extra = nch - base * parts;
    c0 = gw * base + min(gw, extra);
    c1 = c0 + base + (gw < extra ? 1 : 0);
  } else {
    const int hb = nch / kparts, hx = nch - hb * kparts;
    const int h0 = half * hb + min(half, hx);
    const int hn = hb + (half < hx ? 1 : 0);
    const int base = hn / W, extra = hn - base * W;
    c0 = h0 + w * base + min(w, extra);
    c1 = c0 + base + (w < extra ? 1 : 0);
    const int blo = (int)a.page_div.div((uint32_t)(kBlock * h0));
    const int bhi = hn > 0 ? (int)a.page_div.div((uint32_t)(min(len, kBlock * (h0 + hn)) - 1)) + 1 : blo;
    if (bhi > kTableEntries) {
      issue_table(a, b, blo, bhi, threadIdx.x & (kWave - 1), ps.pt);
      ps.blk0 = blo;
    }
  }
  const int M = a.rows;
  const int rec = (int)record_floats(M, HD);
  attend_piece<HD, E, R, true, OutT, COLD, true>(a, lp[w], lq[w], b, kvh, len, kBlock * c0, min(len, kBlock * c1),
                                                 false, s_rec + w * rec, &ps);
  __syncthreads();
  // Thread t folds (row, quad) = (t / kQuads, t % kQuads) of the W records: unnormalised sums of
  // 4 dims, the row's maximum and sum.
  auto fold = [&](int row, int quad, float& mstar, float& l, f32x4& o) {
    mstar = -INFINITY;
#pragma unroll
    for (int k = 0; k < W; ++k) mstar = fmaxf(mstar, s_rec[k * rec + M * HD + row]);
    const float mu = mstar == -INFINITY ? 0.f : mstar;
    l = 0.f;
    o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < W; ++k) {
      const float* rk = s_rec + k * rec;
      const float wk = __builtin_amdgcn_exp2f(rk[M * HD + row] - mu);
      l += wk * rk[M * HD + M + row];
      o += wk * *(const f32x4*)(rk + row * HD + 4 * quad);
    }
  };
  if (!split) {
    for (int t = threadIdx.x; t < M * kQuads; t += W * kWave) {
      const int row = t / kQuads;
      const int quad = t - row * kQuads;
      float mstar, l;
      f32x4 o;
      fold(row, quad, mstar, l, o);
      const float inv = l > 0.f ? 1.f / l : 0.f;
      store_out4<OutT, E>(out_row(a, b, kvh, row) + (int64_t)(4 * quad) * sizeof(OutT), o * inv);
    }
    return;
  }
  if constexpr (S != 1) {
    static_assert(4 * R * kQuads <= W * kWave, "one (row, quad) of the record a thread");
    const int t = threadIdx.x;
    const bool item = t < M * kQuads;
    const int row = t / kQuads;
    const int quad = t - row * kQuads;
    float mstar = -INFINITY, l = 0.f;
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
    // Records nsplit * p + j of the workspace hold the parts of pair p.
    const float* recs = a.part + (int64_t)nsplit * pair * rec;
    float* mine = a.part + ((int64_t)nsplit * pair + half) * rec;
    if (item) {
      fold(row, quad, mstar, l, o);
      uint64_t* d = (uint64_t*)(mine + row * HD + 4 * quad);
      __hip_atomic_store(d, __builtin_bit_cast(uint64_t, float2{o[0], o[1]}), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(d + 1, __builtin_bit_cast(uint64_t, float2{o[2], o[3]}), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (quad == 0) {
        __hip_atomic_store((uint32_t*)(mine + M * HD + row), __builtin_bit_cast(uint32_t, mstar), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store((uint32_t*)(mine + M * HD + M + row), __builtin_bit_cast(uint32_t, l), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
    __syncthreads();
    if (t == 0) {
      int32_t* count = a.ctrl + BARQ_KV_CTRL_PAIR_WORD(pair);
      const int before = __hip_atomic_fetch_add(count, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == kparts - 1) __hip_atomic_store(count, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      s_arrived = before;
    }
    __syncthreads();
    if (s_arrived != kparts - 1 || !item) return;
    // The pair's records, folded in the parts' order whichever workgroup came last (the same bits
    // every call): NS slots' loads issued at once, slots past the pair's parts re-reading its last.
    auto gather_fold = [&](auto ns, float& lsum, f32x4& osum) {
      constexpr int NS = decltype(ns)::value;
      float mm[NS], ll[NS];
      f32x4 oo[NS];
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        if (NS == 2 && j == half) continue;  // two parts: only the other one's record
        const float* rj = recs + (int64_t)min(j, kparts - 1) * rec;
        const uint64_t* e = (const uint64_t*)(rj + row * HD + 4 * quad);
        const float2 o01 = __builtin_bit_cast(float2, __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        const float2 o23 =
            __builtin_bit_cast(float2, __hip_atomic_load(e + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        oo[j] = f32x4{o01.x, o01.y, o23.x, o23.y};
        mm[j] = __builtin_bit_cast(
            float, __hip_atomic_load((const uint32_t*)(rj + M * HD + row), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
        ll[j] = __builtin_bit_cast(float, __hip_atomic_load((const uint32_t*)(rj + M * HD + M + row),
                                                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
      }
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        if (j == half) {
          mm[j] = mstar;
          ll[j] = l;
          oo[j] = o;
        } else if (j >= kparts) {
          mm[j] = -INFINITY;
          ll[j] = 0.f;
          oo[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
      float mboth = -INFINITY;
#pragma unroll
      for (int j = 0; j < NS; ++j) mboth = fmaxf(mboth, mm[j]);
      const float mu = mboth == -INFINITY ? 0.f : mboth;
      lsum = 0.f;
      osum = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < NS; ++j) {
        const float wj = __builtin_amdgcn_exp2f(mm[j] - mu);
        lsum += wj * ll[j];
        osum += wj * oo[j];
      }
    };
    float lsum;
    f32x4 osum;
    if (S == 2 || kparts == 2)
      gather_fold(std::integral_constant<int, 2>{}, lsum, osum);
    else if (S != kSplitLong || kparts <= kMaxSplit)
      gather_fold(std::integral_constant<int, (S == 2 ? 2 : kMaxSplit)>{}, lsum, osum);
    else
      gather_fold(std::integral_constant<int, (S == kSplitLong ? kMaxSplitLong : 2)>{}, lsum, osum);
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    store_out4<OutT, E>(out_row(a, b, kvh, row) + (int64_t)(4 * quad) * sizeof(OutT), osum * inv);
  }
}

// Merge of one query row's records: one workgroup of NT threads per (row, kv head, batch row).
// Thread (quad, class) folds the records class, class + NT / (HD / 4), ... into a running (max,
// sum, 4 dims) -- every record load is independent -- and the classes are folded through LDS.
// Rows of length 0 get zeros here; pairs inside one range were written by their wave.
template <int HD, int E, typename OutT, int NT>
__global__ __launch_bounds__(NT) void attention_merge_kernel(const AttnArgs a) {
  constexpr int kQuads = HD / 4;
  constexpr int kClasses = NT / kQuads;
  __shared__ int s_len[kMaxBatch];
  __shared__ int s_incl[kMaxBatch];
  __shared__ int s_total;
  __shared__ f32x4 po[NT];
  __shared__ float pm[NT];
  __shared__ float pl[NT];

  const int tid = threadIdx.x;
  const int row = blockIdx.x;
  const int kvh = blockIdx.y;
  const int b = blockIdx.z;
  if (tid < kWave) {
    const int total = scan_rows(a, tid, s_len, s_incl, false);
    if (tid == 0) s_total = total;
  }
  __syncthreads();
  const RangeMap rm = range_map(a, s_total);
  const int nch = (s_len[b] + kBlock - 1) / kBlock;
  const int pair_first = (b > 0 ? s_incl[b - 1] : 0) + kvh * nch;
  if (nch == 0) {
    if (tid < kQuads)
      store_out4<OutT, E>(out_row(a, b, kvh, row) + (int64_t)(4 * tid) * sizeof(OutT), f32x4{0.f, 0.f, 0.f, 0.f});
    return;
  }
  const int r_first = rm.of(pair_first);
  const int r_last = rm.of(pair_first + nch - 1);
  if (r_first == r_last) return;

  const int M = a.rows;
  const int64_t rec = record_floats(M, HD);
  const int64_t p = (int64_t)b * a.kv_heads + kvh;
  const int quad = tid % kQuads;
  const int cls = tid / kQuads;
  float mt = -INFINITY, lt = 0.f;
  f32x4 ot = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int r = r_first + cls; r <= r_last; r += kClasses) {
    const float* rp = a.part + (r + p) * rec;
    const float ms = rp[(int64_t)M * HD + row];
    const float ls = rp[(int64_t)M * HD + M + row];
    const f32x4 os = *(const f32x4*)(rp + (int64_t)row * HD + 4 * quad);
    const float mn = fmaxf(mt, ms);
    const float mu = mn == -INFINITY ? 0.f : mn;
    const float wo = __builtin_amdgcn_exp2f(mt - mu);
    const float ws = __builtin_amdgcn_exp2f(ms - mu);
    lt = lt * wo + ls * ws;
    ot = ot * wo + os * ws;
    mt = mn;
  }
  po[tid] = ot;
  pm[tid] = mt;
  pl[tid] = lt;
  __syncthreads();
  if (tid < kQuads) {
    float mstar = pm[tid];
#pragma unroll
    for (int c = 1; c < kClasses; ++c) mstar = fmaxf(mstar, pm[tid + c * kQuads]);
    const float mu = mstar == -INFINITY ? 0.f : mstar;
    float l = 0.f;
    f32x4 o = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < kClasses; ++c) {
      const float w = __builtin_amdgcn_exp2f(pm[tid + c * kQuads] - mu);
      l += w * pl[tid + c * kQuads];
      o += w * po[tid + c * kQuads];
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    store_out4<OutT, E>(out_row(a, b, kvh, row) + (int64_t)(4 * quad) * sizeof(OutT), o * inv);
  }
}

// Resident workgroups of THREADS threads of a kernel on the current device, at most kMaxWaves
// (cached per instantiation and device; host threads may race on the cache, which only ever
// stores the one value a device gives); `fallback` when the runtime cannot tell.
template <int THREADS, typename K>
int resident_blocks(K kernel, int fallback) {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cached[kMaxDevices];  // 0 = not queried yet
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fallback;
  int blocks = dev >= 0 && dev < kMaxDevices ? cached[dev].load(std::memory_order_relaxed) : 0;
  if (blocks == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, THREADS, 0) != hipSuccess)
      return fallback;
    blocks = std::min(std::max(cus * per_cu, 1), kMaxWaves);
    if (dev >= 0 && dev < kMaxDevices) cached[dev].store(blocks, std::memory_order_relaxed);
  }
  return blocks;
}

// Resident waves of a one-wave-workgroup kernel.
template <typename K>
int resident_waves(K kernel) {
  return resident_blocks<kWave>(kernel, kMaxWaves);
}

template <int HD, int E, int R, bool U, typename OutT, bool COLD>
hipError_t launch_typed(AttnArgs a, bool merge, hipStream_t stream) {
  // Pairs of bounded length, the automatic split, whole-chunk pages, up to 8 query rows (two waves
  // per SIMD keep the accumulators in registers): one workgroup per pair.
  if constexpr (U && R <= 2 && HD <= 128) {
    const int64_t pairs = (int64_t)a.batch * a.kv_heads;
    // Fewer pairs than kPairMinPairs leave CUs idle, but up to kPairMaxChunks a pair one launch
    // still beats the flat pair of launches and its merge (C2 shape at batch 1: 650 positions
    // 16.3 -> 12.6 us, 128 positions 12.8 -> 6.3 us; at 2048 the flat schedule wins, 14.8 against
    // 28.4).
    // Workgroups a pair: as many as are resident at once with the others' (the kernel decides per
    // row how many it uses), at most kMaxSplit; the pair counts in ctrl bound the pairs.
    auto* split_any = attention_pair_kernel<HD, E, R, OutT, COLD, kPairWaves, kSplitAny>;
    const int64_t chunks = (a.max_seq + kBlock - 1) / kBlock;
    const int64_t nsplit =
        pairs > 0 && pairs <= BARQ_KV_CTRL_PAIR_SLOTS && chunks >= 2 * pair_part_chunks<R>()
            ? std::min<int64_t>(kMaxSplit, resident_blocks<kPairWaves * kWave>(split_any, 0) / pairs)
            : 1;
    int64_t max_chunks = R > 1 || pairs < kPairMinPairs        ? kPairMaxChunks
                         : COLD || pairs < 2 * kPairMinPairs ? kPairMaxChunksR1
                                                             : kPairMaxChunksR1Wide;
    if (nsplit > 2) max_chunks = std::min<int64_t>(kTableEntries, std::max(max_chunks, nsplit * kSplitChunksPerPart));
    // Two workgroups a pair halve each one's chunks: 5 to 8 query rows take the bound of up to 4.
    if (nsplit == 2 && R > 1 && pairs >= kPairMinPairs) max_chunks = std::max(max_chunks, kPairMaxChunksR1);
    if (a.range_chunks == 0 && pairs > 0 && chunks <= max_chunks) {
      if (nsplit > 2) {
        hipLaunchKernelGGL(split_any, dim3((unsigned)(nsplit * pairs)), dim3(kPairWaves * kWave), 0, stream, a);
      } else if (nsplit == 2) {
        hipLaunchKernelGGL((attention_pair_kernel<HD, E, R, OutT, COLD, kPairWaves, 2>), dim3((unsigned)(2 * pairs)),
                           dim3(kPairWaves * kWave), 0, stream, a);
      } else {
        hipLaunchKernelGGL((attention_pair_kernel<HD, E, R, OutT, COLD, kPairWaves, 1>), dim3((unsigned)pairs),
                           dim3(kPairWaves * kWave), 0, stream, a);
      }
      return hipGetLastError();
    }
    // Longer rows at small batches (C4 at 32k positions: 34.3 -> 31.1 us against the flat pair of
    // launches): up to kMaxSplitLong workgroups a pair, each part's blocks in a window of its own.
    if (a.range_chunks == 0 && pairs > 0 && pairs <= BARQ_KV_CTRL_PAIR_SLOTS) {
      auto* split_long = attention_pair_kernel<HD, E, R, OutT, COLD, kPairWaves, kSplitLong>;
      const int64_t nlong =
          std::min<int64_t>(kMaxSplitLong, resident_blocks<kPairWaves * kWave>(split_long, 0) / pairs);
      if (nlong > 2 && chunks <= nlong * kLongChunksPerPart) {
        hipLaunchKernelGGL(split_long, dim3((unsigned)(nlong * pairs)), dim3(kPairWaves * kWave), 0, stream, a);
        return hipGetLastError();
      }
    }
  }
  auto* k = attention_flat_kernel<HD, E, R, U, OutT, COLD>;
  a.waves = resident_waves(k);
  hipLaunchKernelGGL(k, dim3((unsigned)a.waves), dim3(kWave), 0, stream, a);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || !merge) return err;
  // Fewer merge workgroups than CUs (few long pairs, many records each): 1024 threads each.
  if ((int64_t)a.rows * a.kv_heads * a.batch < kMergeWideBelow)
    hipLaunchKernelGGL((attention_merge_kernel<HD, E, OutT, kMergeWide>),
                       dim3((unsigned)a.rows, (unsigned)a.kv_heads, (unsigned)a.batch), dim3(kMergeWide), 0, stream, a);
  else
    hipLaunchKernelGGL((attention_merge_kernel<HD, E, OutT, kThreads>),
                       dim3((unsigned)a.rows, (unsigned)a.kv_heads, (unsigned)a.batch), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template <int HD, int E, int R, bool U, bool COLD>
hipError_t launch_out(const AttnArgs& a, bool out_f32, bool merge, hipStream_t stream) {
  return out_f32 ? launch_typed<HD, E, R, U, float, COLD>(a, merge, stream)
                 : launch_typed<HD, E, R, U, uint16_t, COLD>(a, merge, stream);
}

template <int HD, int E, bool U, bool COLD>
hipError_t launch_rows(const AttnArgs& a, bool out_f32, bool merge, hipStream_t stream) {
  const int groups = (a.rows + 3) / 4;
  return groups == 1   ? launch_out<HD, E, 1, U, COLD>(a, out_f32, merge, stream)
         : groups == 2 ? launch_out<HD, E, 2, U, COLD>(a, out_f32, merge, stream)
                       : launch_out<HD, E, 4, U, COLD>(a, out_f32, merge, stream);
}

template <int HD, int E>
hipError_t launch_pages(const AttnArgs& a, bool uniform, bool cold, bool out_f32, bool merge, hipStream_t stream) {
  if constexpr (HD == 256) {  // two-byte pages only (the caller refuses quantised pools)
    return uniform ? launch_rows<HD, E, true, false>(a, out_f32, merge, stream)
                   : launch_rows<HD, E, false, false>(a, out_f32, merge, stream);
  } else {
    if (cold)  // quantised pools: page_size a multiple of 16 (checked by the caller)
      return launch_rows<HD, E, true, true>(a, out_f32, merge, stream);
    return uniform ? launch_rows<HD, E, true, false>(a, out_f32, merge, stream)
                   : launch_rows<HD, E, false, false>(a, out_f32, merge, stream);
  }
}

template <int E>
hipError_t launch_dtype(const AttnArgs& a, int head_dim, bool uniform, bool cold, bool out_f32, bool merge,
                        hipStream_t stream) {
  return head_dim == 64    ? launch_pages<64, E>(a, uniform, cold, out_f32, merge, stream)
         : head_dim == 128 ? launch_pages<128, E>(a, uniform, cold, out_f32, merge, stream)
                           : launch_pages<256, E>(a, uniform, cold, out_f32, merge, stream);
}

struct AttnPlan {
  int64_t rows;
  int64_t max_seq;
  int64_t range_chunks;  // 0: automatic
  int64_t records;       // record slots the workspace holds
  int64_t bytes;
};

// Validates the geometry and sizes the workspace.  max_seq bounds every row's length (0: the
// pool's capacity); split_tokens fixes the positions of a range (rounded up to 16; 0: the flat
// schedule's own, total / resident waves).
int plan_attention(const barq_kv_pool* pool, int64_t batch, int64_t q_heads, int64_t tokens,
                   int64_t max_seq, int64_t split_tokens, AttnPlan* plan) {
  if (!pool || pool->elem_bytes != 2 || (pool->head_dim != 64 && pool->head_dim != 128 && pool->head_dim != 256) || pool->kv_heads <= 0 ||
      pool->page_size <= 0 || pool->max_blocks <= 0 || pool->num_pages <= 0 ||
      pool->num_pages > INT32_MAX || pool->max_batch <= 0)
    return BARQ_KV_ERR_INVALID;
  if (batch < 0 || batch > pool->max_batch || batch > kMaxBatch || tokens <= 0 || q_heads <= 0 ||
      q_heads % pool->kv_heads != 0)
    return BARQ_KV_ERR_INVALID;
  const int64_t rows = (q_heads / pool->kv_heads) * tokens;
  if (rows > kMaxRows) return BARQ_KV_ERR_INVALID;
  const int64_t capacity = pool->max_blocks * pool->page_size;
  const int64_t row_bytes = pool->kv_heads * pool->head_dim * 2;
  if (max_seq <= 0 || max_seq > capacity) max_seq = capacity;
  // Lane offsets within a page are 32-bit; chunk indices of the whole schedule fit 31 bits.
  const int64_t pairs = batch * pool->kv_heads;
  const int64_t max_chunks = pairs * ((max_seq + kBlock - 1) / kBlock);
  if (capacity > INT32_MAX / 2 || row_bytes * pool->page_size > INT32_MAX / 2 ||
      max_chunks > INT32_MAX / 2 || pool->kv_heads > 65535)
    return BARQ_KV_ERR_INVALID;
  if (split_tokens < 0 || split_tokens > INT32_MAX / 2) return BARQ_KV_ERR_INVALID;
  const int64_t chunks = split_tokens > 0 ? (split_tokens + kBlock - 1) / kBlock : 0;
  // Ranges: at most kMaxWaves automatically, else as many as the fixed range length gives.
  const int64_t ranges = chunks > 0 ? (max_chunks + chunks - 1) / chunks : kMaxWaves;
  plan->rows = rows;
  plan->max_seq = max_seq;
  plan->range_chunks = chunks;
  plan->records = ranges + pairs;
  plan->bytes = plan->records * record_floats(rows, pool->head_dim) * 4;
  return BARQ_KV_OK;
}

}  // namespace

extern "C" {

int64_t barq_kv_attention_workspace_bytes(const barq_kv_pool* pool, int64_t batch,
                                          int64_t q_heads, int64_t tokens, int64_t max_seq,
                                          int64_t split_tokens) {
  AttnPlan plan;
  if (plan_attention(pool, batch, q_heads, tokens, max_seq, split_tokens, &plan) != BARQ_KV_OK)
    return -1;
  return plan.bytes;
}

}  // extern "C"

namespace {

int decode_attention(const barq_kv_pool* pool, const barq_kv_cold* cold, const void* query, int64_t batch,
                     int64_t q_heads, int64_t tokens, int64_t q_stride_b, int64_t q_stride_h,
                     int64_t q_stride_t, void* out, int64_t out_stride_b, int64_t out_stride_h,
                     int64_t out_stride_t, float scale, int64_t max_seq, int64_t split_tokens, int64_t flags,
                     void* workspace, int64_t workspace_bytes, void* stream) {
  AttnPlan plan;
  const int rc = plan_attention(pool, batch, q_heads, tokens, max_seq, split_tokens, &plan);
  if (rc != BARQ_KV_OK) return rc;
  if (flags & ~(int64_t)(BARQ_KV_ATTN_FP16 | BARQ_KV_ATTN_OUT_F32)) return BARQ_KV_ERR_INVALID;
  if (batch == 0) return BARQ_KV_OK;
  const int64_t out_elem = (flags & BARQ_KV_ATTN_OUT_F32) ? 4 : 2;
  if (!query || !out || !workspace || workspace_bytes < plan.bytes || !pool->key_pages ||
      !pool->value_pages || !pool->block_table || !pool->seq_lens || !pool->ctrl)
    return BARQ_KV_ERR_INVALID;
  // 16-byte query rows and 4-element output runs must be aligned for the vector accesses.
  const int64_t qs[3] = {q_stride_b, q_stride_h, q_stride_t};
  const int64_t os[3] = {out_stride_b, out_stride_h, out_stride_t};
  for (int i = 0; i < 3; ++i) {
    if (qs[i] < 0 || qs[i] % 8 != 0 || os[i] < 0 || os[i] % 8 != 0) return BARQ_KV_ERR_INVALID;
  }
  if (((uintptr_t)query | (uintptr_t)pool->key_pages | (uintptr_t)pool->value_pages) % 16 != 0 ||
      (uintptr_t)out % (out_elem * 4) != 0 || (uintptr_t)workspace % 16 != 0)
    return BARQ_KV_ERR_INVALID;

  AttnArgs a;
  a.kpages = (const char*)pool->key_pages;
  a.vpages = (const char*)pool->value_pages;
  a.block_table = pool->block_table;
  a.seq_lens = pool->seq_lens;
  a.errors = pool->ctrl + BARQ_KV_CTRL_ERRORS;
  a.ctrl = pool->ctrl;
  a.head_bytes = (int32_t)(pool->head_dim * 2);
  a.row_bytes = (int32_t)(pool->kv_heads * a.head_bytes);
  a.page_bytes = pool->page_size * (int64_t)a.row_bytes;
  a.q_sb = q_stride_b * 2;
  a.q_sh = q_stride_h * 2;
  a.q_st = q_stride_t * 2;
  a.o_sb = out_stride_b * out_elem;
  a.o_sh = out_stride_h * out_elem;
  a.o_st = out_stride_t * out_elem;
  a.q = (const char*)query;
  a.out = (char*)out;
  a.part = (float*)workspace;
  a.page_div = FastDiv::make((uint32_t)pool->page_size);
  a.num_pages = (int32_t)pool->num_pages;
  a.max_blocks = (int32_t)pool->max_blocks;
  a.page_size = (int32_t)pool->page_size;
  a.kv_heads = (int32_t)pool->kv_heads;
  a.group = (int32_t)(q_heads / pool->kv_heads);
  a.tokens = (int32_t)tokens;
  a.rows = (int32_t)plan.rows;
  a.batch = (int32_t)batch;
  a.max_seq = (int32_t)plan.max_seq;
  a.range_chunks = (int32_t)plan.range_chunks;
  a.waves = kMaxWaves;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.kcodes = a.vcodes = a.kscales = a.vscales = nullptr;
  a.num_cold = 0;

  const bool uniform = pool->page_size % kBlock == 0;
  if (cold && pool->head_dim == 256) return BARQ_KV_ERR_INVALID;  // quantised pools: head sizes 64, 128
  if (cold) {
    const int64_t want = (flags & BARQ_KV_ATTN_FP16) ? BARQ_KV_FP16 : BARQ_KV_BF16;
    if (!uniform || cold->element_type != want || !cold->key_codes || !cold->value_codes || !cold->key_scales ||
        !cold->value_scales || cold->num_cold < 1 || cold->num_cold > INT32_MAX - 2 ||
        ((uintptr_t)cold->key_codes | (uintptr_t)cold->value_codes | (uintptr_t)cold->key_scales) % 8 != 0)
      return BARQ_KV_ERR_INVALID;
    a.kcodes = (const uint8_t*)cold->key_codes;
    a.vcodes = (const uint8_t*)cold->value_codes;
    a.kscales = (const uint8_t*)cold->key_scales;
    a.vscales = (const uint8_t*)cold->value_scales;
    a.num_cold = (int32_t)cold->num_cold;
  }
  const bool out_f32 = (flags & BARQ_KV_ATTN_OUT_F32) != 0;
  const hipError_t err =
      (flags & BARQ_KV_ATTN_FP16)
          ? launch_dtype<kF16>(a, (int)pool->head_dim, uniform, cold != nullptr, out_f32, true, (hipStream_t)stream)
          : launch_dtype<kBF16>(a, (int)pool->head_dim, uniform, cold != nullptr, out_f32, true, (hipStream_t)stream);
  return err == hipSuccess ? BARQ_KV_OK : BARQ_KV_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int barq_kv_decode_attention(const barq_kv_pool* pool, const void* query, int64_t batch,
                             int64_t q_heads, int64_t tokens, int64_t q_stride_b,
                             int64_t q_stride_h, int64_t q_stride_t, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, int64_t out_stride_t,
                             float scale, int64_t max_seq, int64_t split_tokens, int64_t flags,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  return decode_attention(pool, nullptr, query, batch, q_heads, tokens, q_stride_b, q_stride_h, q_stride_t, out,
                          out_stride_b, out_stride_h, out_stride_t, scale, max_seq, split_tokens, flags, workspace,
                          workspace_bytes, stream);
}

// Workspace of barq_kv_decode_attention_noalloc: one static array per GPU.  Host code never
// passes `scratch` itself (in host code the name is a stand-in, not a device address); the
// kernels get the address hipGetSymbolAddress resolves on each device.
static __device__ __align__(256) unsigned char scratch[BARQ_KV_SCRATCH_BYTES];

int barq_kv_decode_attention_noalloc(const barq_kv_pool* pool, const void* query, int64_t batch,
                                     int64_t q_heads, int64_t tokens, int64_t q_stride_b,
                                     int64_t q_stride_h, int64_t q_stride_t, void* out,
                                     int64_t out_stride_b, int64_t out_stride_h,
                                     int64_t out_stride_t, float scale, int64_t max_seq,
                                     int64_t split_tokens, int64_t flags, void* stream) {
  AttnPlan plan;
  const int rc = plan_attention(pool, batch, q_heads, tokens, max_seq, split_tokens, &plan);
  if (rc != BARQ_KV_OK) return rc;
  if (plan.bytes > BARQ_KV_SCRATCH_BYTES) return BARQ_KV_ERR_SCRATCH;
  // The array's address on the current device, resolved on the first call there.
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addr[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return BARQ_KV_ERR_LAUNCH;
  void* ptr = addr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr) return BARQ_KV_ERR_LAUNCH;
    addr[dev].store(ptr, std::memory_order_release);
  }
  return decode_attention(pool, nullptr, query, batch, q_heads, tokens, q_stride_b, q_stride_h, q_stride_t, out,
                          out_stride_b, out_stride_h, out_stride_t, scale, max_seq, split_tokens, flags, ptr,
                          BARQ_KV_SCRATCH_BYTES, stream);
}

int barq_kv_decode_attention_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, const void* query,
                                  int64_t batch, int64_t q_heads, int64_t tokens, int64_t q_stride_b,
                                  int64_t q_stride_h, int64_t q_stride_t, void* out, int64_t out_stride_b,
                                  int64_t out_stride_h, int64_t out_stride_t, float scale, int64_t max_seq,
                                  int64_t split_tokens, int64_t flags, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
  if (!cold) return BARQ_KV_ERR_INVALID;
  return decode_attention(pool, cold, query, batch, q_heads, tokens, q_stride_b, q_stride_h, q_stride_t, out,
                          out_stride_b, out_stride_h, out_stride_t, scale, max_seq, split_tokens, flags, workspace,
                          workspace_bytes, stream);
}

}  // extern "C"
