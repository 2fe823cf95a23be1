// fp8 cold store of a page pool for MI355X (gfx950), behind the C ABI of include/barq_kv.h:
// blocks behind a row's residual window are quantised (barq_kv_compress) to OCP FP8 E4M3 codes
// with power-of-two (E8M0) scales -- keys per channel over the page's tokens, values per token
// over head_dim, KIVI's grouping -- and dequantised on the way out (barq_kv_gather_cold).
//
// Power-of-two scales make scaling exact, so a code depends only on its element and its group's
// largest finite magnitude, and a dequantised value is exactly code * 2^e before the final
// rounding to the pool's element type: the same numbers on every run and every device.
//
// The reference plans this path (IMPLEMENTATION_PLAN.md:106-129: quantized KV storage, a
// full-precision residual window, dequant-on-read) and has no implementation.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <climits>

#include "barq_kv.h"
#include <atomic>

#include "barq_kv_commit.h"
#include "barq_kv_fp8.h"
#include "fastdiv.h"

namespace {

// s_waitcnt vmcnt(K), the other counters left alone (vmcnt bits 3:0, expcnt 6:4, lgkmcnt 11:8).
template <int K>
__device__ __forceinline__ void wait_vm() {
  static_assert(K >= 0 && K < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt(K | (0x7 << 4) | (0xF << 8));
}

constexpr int kThreads = 256;
constexpr int kWave = 64;
constexpr int kWaves = kThreads / kWave;
constexpr int kMaxTokenHeads = 4096;  // page_size * kv_heads: a compress workgroup's value maxima
constexpr int kMaxChannels = 16384;   // kv_heads * head_dim: a compress workgroup's key exponents
constexpr int kUnroll = 4;            // vectors in flight per gather thread
constexpr int kGatherThreads = 256;   // a gather workgroup: 4 waves
constexpr int64_t kI32Max = 0x7fffffffLL;

__device__ __forceinline__ int checked_id(int id, int64_t n) { return (id >= 0 && (int64_t)id < n) ? id : -1; }

__device__ __forceinline__ int ceil_div_fd(int n, const FastDiv& d) {
  return n <= 0 ? 0 : (int)d.div((uint32_t)(n + (int)d.d - 1));
}

__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int up = __shfl_up(v, o, kWave);
    if (lane >= o) v += up;
  }
  return v;
}

// Exclusive prefix sum over the workgroup; *total gets the sum.  Every thread must call it.
__device__ __forceinline__ int block_exclusive_scan(int v, int* lds, int* total) {
  const int wave = threadIdx.x / kWave;
  const int incl = wave_incl_scan(v);
  if ((threadIdx.x & (kWave - 1)) == kWave - 1) lds[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int t = lds[w];
    if (w < wave) before += t;
    all += t;
  }
  __syncthreads();
  *total = all;
  return before + incl - v;
}

using barq_fp8::codes_normal;
using barq_fp8::e4m3_decode;
using barq_fp8::e4m3_encode;
using barq_fp8::e4m3_encode4;
using barq_fp8::Elem;
using barq_fp8::fast_pair;
using barq_fp8::finite_abs;
using barq_fp8::group_exponent;
using barq_fp8::scale_fast;
using barq_fp8::spread_hi;
using barq_fp8::spread_lo;

struct ColdPtrs {
  uint8_t* codes[2];   // key, value
  uint8_t* key_scales;
  uint8_t* value_scales;
  int32_t* free_cold;
  int32_t* shares;     // references beyond the first, or null
  int64_t num_cold;
  int32_t window;
};

// ---------------------------------------------------------------------------------------------
// Compress: workgroup per row.  quantise_page serves any geometry; quantise_regs below (one
// round trip of loads per page) the common two-byte ones.
// ---------------------------------------------------------------------------------------------

struct CompressArgs {
  barq_kv_pool p;
  ColdPtrs c;
  int32_t batch;
  int32_t ahead;       // tokens the rows are about to receive: quantise for lengths + ahead
  FastDiv div_page;
  FastDiv div_dim;     // head_dim
  FastDiv div_groups;  // kv_heads * head_dim / VE vectors per token
};

template <int BYTES>
struct RawC;
template <>
struct RawC<16> { using T = uint32_t __attribute__((ext_vector_type(4))); };
template <>
struct RawC<8> { using T = uint32_t __attribute__((ext_vector_type(2))); };
template <>
struct RawC<4> { using T = uint32_t; };
template <>
struct RawC<2> { using T = uint16_t; };
template <>
struct RawC<1> { using T = uint8_t; };

// VE elements of one token, as floats, from a page.
template <int KIND, int VE>
struct Lanes {
  using Bits = typename Elem<KIND>::Bits;
  using Raw = typename RawC<VE * (int)sizeof(Bits)>::T;
  union U {
    Raw v;
    Bits e[VE];
  };
  __device__ static void load(const Bits* src, float* out) {
    U u;
    u.v = *(const Raw*)src;
#pragma unroll
    for (int e = 0; e < VE; ++e) out[e] = Elem<KIND>::to_float(u.e[e]);
  }
};

template <int VE>
struct CodeVec {
  using Raw = typename RawC<VE>::T;
  union U {
    Raw v;
    uint8_t b[VE];
  };
};

// Quantise hot page hp into cold page cp (keys per channel, values per (token, head)), in vectors
// of VE elements along head_dim: maxima first (keys: a thread's channels over the page's tokens;
// values: a thread's (token, head) groups over head_dim), exponents to LDS, then codes.
template <int KIND, int VE>
__device__ void quantise_page(const CompressArgs& a, int hp, int cp, int8_t* s_kexp, int8_t* s_vexp) {
  using Bits = typename Elem<KIND>::Bits;
  const barq_kv_pool& p = a.p;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim, C = H * D;
  const Bits* __restrict__ kp = (const Bits*)p.key_pages + (int64_t)hp * P * C;
  const Bits* __restrict__ vp = (const Bits*)p.value_pages + (int64_t)hp * P * C;
  const int groups = C / VE;
  for (int g = threadIdx.x; g < groups; g += kThreads) {
    float m[VE];
#pragma unroll
    for (int e = 0; e < VE; ++e) m[e] = 0.0f;
#pragma unroll 4
    for (int t = 0; t < P; ++t) {
      float x[VE];
      Lanes<KIND, VE>::load(kp + (int64_t)t * C + g * VE, x);
#pragma unroll
      for (int e = 0; e < VE; ++e) m[e] = fmaxf(m[e], finite_abs(x[e]));
    }
    typename CodeVec<VE>::U sc;
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      const int ex = group_exponent(m[e]);
      s_kexp[g * VE + e] = (int8_t)ex;
      sc.b[e] = (uint8_t)(ex + 127);
    }
    *(typename CodeVec<VE>::Raw*)(a.c.key_scales + (int64_t)cp * C + g * VE) = sc.v;
  }
  const int dv = D / VE;
  for (int th = threadIdx.x; th < P * H; th += kThreads) {
    const Bits* src = vp + (int64_t)th * D;  // token t = th / H, head h = th % H: contiguous
    float m = 0.0f;
#pragma unroll 4
    for (int k = 0; k < dv; ++k) {
      float x[VE];
      Lanes<KIND, VE>::load(src + k * VE, x);
#pragma unroll
      for (int e = 0; e < VE; ++e) m = fmaxf(m, finite_abs(x[e]));
    }
    const int ex = group_exponent(m);
    s_vexp[th] = (int8_t)ex;
    a.c.value_scales[(int64_t)cp * P * H + th] = (uint8_t)(ex + 127);
  }
  __syncthreads();
  uint8_t* __restrict__ kc = a.c.codes[0] + (int64_t)cp * P * C;
  uint8_t* __restrict__ vc = a.c.codes[1] + (int64_t)cp * P * C;
#pragma unroll 2
  for (int v = threadIdx.x; v < P * groups; v += kThreads) {
    const int t = (int)a.div_groups.div((uint32_t)v);
    const int g = v - t * groups;
    const int ch = g * VE;
    const int th = t * H + (int)a.div_dim.div((uint32_t)ch);
    const int64_t at = (int64_t)t * C + ch;
    float xk[VE], xv[VE];
    Lanes<KIND, VE>::load(kp + at, xk);
    Lanes<KIND, VE>::load(vp + at, xv);
    const int ve = s_vexp[th];
    typename CodeVec<VE>::U ck, cv;
    if constexpr (VE % 4 == 0) {
      uint32_t wk[VE / 4], wv[VE / 4];
#pragma unroll
      for (int q = 0; q < VE / 4; ++q) {
        const int e = 4 * q;
        wk[q] = e4m3_encode4(ldexpf(xk[e], -(int)s_kexp[ch + e]), ldexpf(xk[e + 1], -(int)s_kexp[ch + e + 1]),
                             ldexpf(xk[e + 2], -(int)s_kexp[ch + e + 2]), ldexpf(xk[e + 3], -(int)s_kexp[ch + e + 3]));
        wv[q] = e4m3_encode4(ldexpf(xv[e], -ve), ldexpf(xv[e + 1], -ve), ldexpf(xv[e + 2], -ve), ldexpf(xv[e + 3], -ve));
      }
      __builtin_memcpy(ck.b, wk, VE);
      __builtin_memcpy(cv.b, wv, VE);
    } else {
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        ck.b[e] = (uint8_t)e4m3_encode(ldexpf(xk[e], -(int)s_kexp[ch + e]));
        cv.b[e] = (uint8_t)e4m3_encode(ldexpf(xv[e], -ve));
      }
    }
    *(typename CodeVec<VE>::Raw*)(kc + at) = ck.v;
    *(typename CodeVec<VE>::Raw*)(vc + at) = cv.v;
  }
}

template <int KIND, int VE>
__global__ void __launch_bounds__(kThreads) compress_kernel(const CompressArgs a) {
  __shared__ int lds_scan[kWaves];
  __shared__ int s_blocks[kThreads];
  __shared__ int s_cold;
  __shared__ int8_t s_vexp[kMaxTokenHeads];
  __shared__ int8_t s_kexp[kMaxChannels];
  const barq_kv_pool& p = a.p;
  const int r = blockIdx.x;
  const int mb = (int)p.max_blocks;
  const int len = p.seq_lens[r] + a.ahead;
  const int old_len = len - a.c.window;
  const int jmax = min(old_len > 0 ? (int)a.div_page.div((uint32_t)old_len) : 0,
                       min(ceil_div_fd(max(p.high_water[r], len), a.div_page), mb));
  int32_t* row = p.block_table + (int64_t)r * mb;
  int err = 0;
  for (int j0 = 0; j0 < jmax; j0 += kThreads) {
    const int j = j0 + (int)threadIdx.x;
    int hot = 0;
    if (j < jmax) {
      const int page = checked_id(row[j], p.num_pages);
      hot = page >= 0 && (!p.page_shares || p.page_shares[page] == 0);
    }
    int count = 0;
    const int k = block_exclusive_scan(hot, lds_scan, &count);
    if (hot) s_blocks[k] = j;
    __syncthreads();
    for (int q = 0; q < count; ++q) {
      const int jb = s_blocks[q];
      if (threadIdx.x == 0) {
        int cp = -1;
        const int before = atomicSub(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], 1);
        if (before <= 0 || (int64_t)before > a.c.num_cold) {
          atomicAdd(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], 1);
          err |= before <= 0 ? BARQ_KV_ERRBIT_POOL_EXHAUSTED : BARQ_KV_ERRBIT_BAD_INDEX;
        } else {
          cp = checked_id(a.c.free_cold[before - 1], a.c.num_cold);
          if (cp < 0) err |= BARQ_KV_ERRBIT_BAD_INDEX;
        }
        s_cold = cp;
      }
      __syncthreads();
      const int cp = s_cold;
      const int hp = row[jb];
      if (cp >= 0) {  // uniform
        quantise_page<KIND, VE>(a, hp, cp, s_kexp, s_vexp);
        __syncthreads();  // every thread has read the hot page before it is released
        if (threadIdx.x == 0) {
          row[jb] = BARQ_KV_COLD_ENTRY(cp);
          const int slot = atomicAdd(&p.ctrl[BARQ_KV_CTRL_FREE_TOP], 1);
          if (slot < p.num_pages) p.free_pages[slot] = hp;
          else err |= BARQ_KV_ERRBIT_BAD_INDEX;
        }
      }
      __syncthreads();
    }
  }
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// Register-resident compress for 16-byte vectors of 2-byte elements, when a token's G = C / 8
// vectors divide the workgroup (G | 256), a page holds NV * 256 vectors and D / 8 is a power of
// two: thread t holds vectors t + 256 i (i < NV) of a page's K and V -- channel group t % G of
// tokens t / G + i * 256 / G -- so a page costs one round trip of loads, issued (for a row's first
// block) while the cold pages are popped.  Key maxima over the page's tokens combine the 256 / G
// threads of a channel group through LDS; value maxima over a (token, head) combine the head's
// D / 8 adjacent lanes with shuffles.  The codes and scales are quantise_page's: maxima of finite
// magnitudes, group_exponent, e4m3_encode of x * 2^-e.  A row's blocks take the cold pages its one
// pop reserves in block order (free_cold[top - 1], [top - 2], ...), and their hot pages go back
// with one push, in block order.
constexpr int kRegsMaxChannels = 2048;  // C = G * 8 with G | 256

template <int KIND, int NV>
struct PageRegs {
  using Raw = typename RawC<16>::T;
  Raw k[NV], v[NV];

  __device__ void load(const barq_kv_pool& p, int hp, int C) {
    const Raw* kp = (const Raw*)((const char*)p.key_pages + (int64_t)hp * p.page_size * C * 2);
    const Raw* vp = (const Raw*)((const char*)p.value_pages + (int64_t)hp * p.page_size * C * 2);
#pragma unroll
    for (int i = 0; i < NV; ++i) k[i] = kp[threadIdx.x + kThreads * i];
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = vp[threadIdx.x + kThreads * i];
  }
  __device__ static float elem(const Raw& w, int e) {
    return Elem<KIND>::to_float((uint16_t)(w[e >> 1] >> (16 * (e & 1))));
  }
};

template <int KIND, int NV>
__device__ void quantise_regs(const CompressArgs& a, const PageRegs<KIND, NV>& pg, int cp, float* s_red,
                              int8_t* s_kexp) {
  using Regs = PageRegs<KIND, NV>;
  const barq_kv_pool& p = a.p;
  const int t = threadIdx.x;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim, C = H * D;
  const int G = C / 8, VD = D / 8, R = kThreads / G;  // R threads share a channel group
  const int g = t % G;
  // key maxima over the page's tokens, per channel
  float mk[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) mk[e] = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) mk[e] = fmaxf(mk[e], finite_abs(Regs::elem(pg.k[i], e)));
#pragma unroll
  for (int e = 0; e < 8; ++e) s_red[t * 8 + e] = mk[e];
  __syncthreads();
  if (t < G) {
    typename CodeVec<8>::U sc;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float m = s_red[t * 8 + e];
      for (int q = 1; q < R; ++q) m = fmaxf(m, s_red[(t + q * G) * 8 + e]);
      const int ex = group_exponent(m);
      s_kexp[t * 8 + e] = (int8_t)ex;
      sc.b[e] = (uint8_t)(ex + 127);
    }
    *(typename CodeVec<8>::Raw*)(a.c.key_scales + (int64_t)cp * C + t * 8) = sc.v;
  }
  __syncthreads();
  int kex[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) kex[e] = s_kexp[g * 8 + e];
  uint8_t* __restrict__ kc = a.c.codes[0] + (int64_t)cp * P * C;
  uint8_t* __restrict__ vc = a.c.codes[1] + (int64_t)cp * P * C;
  const int h = g / VD;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int tok = t / G + i * R;
    // value maxima over (token, head): the head's VD adjacent lanes
    float mv = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) mv = fmaxf(mv, finite_abs(Regs::elem(pg.v[i], e)));
    for (int o = 1; o < VD; o <<= 1) mv = fmaxf(mv, __shfl_xor(mv, o, kWave));
    const int ve = group_exponent(mv);
    if (g % VD == 0) a.c.value_scales[((int64_t)cp * P + tok) * H + h] = (uint8_t)(ve + 127);
    typename CodeVec<8>::U ck, cv;
    uint32_t wk[2], wv[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int e = 4 * q;
      wk[q] = e4m3_encode4(ldexpf(Regs::elem(pg.k[i], e), -kex[e]), ldexpf(Regs::elem(pg.k[i], e + 1), -kex[e + 1]),
                           ldexpf(Regs::elem(pg.k[i], e + 2), -kex[e + 2]),
                           ldexpf(Regs::elem(pg.k[i], e + 3), -kex[e + 3]));
      wv[q] = e4m3_encode4(ldexpf(Regs::elem(pg.v[i], e), -ve), ldexpf(Regs::elem(pg.v[i], e + 1), -ve),
                           ldexpf(Regs::elem(pg.v[i], e + 2), -ve), ldexpf(Regs::elem(pg.v[i], e + 3), -ve));
    }
    __builtin_memcpy(ck.b, wk, 8);
    __builtin_memcpy(cv.b, wv, 8);
    const int64_t at = (int64_t)tok * C + g * 8;
    *(typename CodeVec<8>::Raw*)(kc + at) = ck.v;
    *(typename CodeVec<8>::Raw*)(vc + at) = cv.v;
  }
}

template <int KIND, int NV>
__global__ void __launch_bounds__(kThreads) compress_regs_kernel(const CompressArgs a) {
  __shared__ int lds_scan[kWaves];
  __shared__ int s_blocks[kThreads];
  __shared__ int s_pages[kThreads];
  __shared__ int s_cold[kThreads];
  __shared__ int s_avail, s_top, s_slot;
  __shared__ float s_red[kThreads * 8];
  __shared__ int8_t s_kexp[kRegsMaxChannels];
  const barq_kv_pool& p = a.p;
  const int tid = threadIdx.x;
  const int r = blockIdx.x;
  const int mb = (int)p.max_blocks;
  const int C = (int)(p.kv_heads * p.head_dim);
  const int len = p.seq_lens[r] + a.ahead;
  const int old_len = len - a.c.window;
  const int jmax = min(old_len > 0 ? (int)a.div_page.div((uint32_t)old_len) : 0,
                       min(ceil_div_fd(max(p.high_water[r], len), a.div_page), mb));
  int32_t* row = p.block_table + (int64_t)r * mb;
  int err = 0;
  for (int j0 = 0; j0 < jmax; j0 += kThreads) {
    const int j = j0 + tid;
    int hot = 0, page = -1;
    if (j < jmax) {
      page = checked_id(row[j], p.num_pages);
      hot = page >= 0 && (!p.page_shares || p.page_shares[page] == 0);
    }
    int count = 0;
    const int k = block_exclusive_scan(hot, lds_scan, &count);
    if (hot) {
      s_blocks[k] = j;
      s_pages[k] = page;
    }
    __syncthreads();
    if (count == 0) continue;  // uniform
    PageRegs<KIND, NV> pg;
    pg.load(p, s_pages[0], C);  // in flight while the cold pages are reserved
    if (tid == 0) {
      const int before = atomicSub(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], count);
      int avail = 0;
      if ((int64_t)before > a.c.num_cold) {
        atomicAdd(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], count);
        err |= BARQ_KV_ERRBIT_BAD_INDEX;
      } else {
        avail = min(max(before, 0), count);
        if (avail < count) {
          atomicAdd(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], count - avail);
          err |= BARQ_KV_ERRBIT_POOL_EXHAUSTED;
        }
      }
      s_avail = avail;
      s_top = before;
    }
    __syncthreads();
    const int avail = s_avail;
    if (tid < avail) {
      const int cp = checked_id(a.c.free_cold[s_top - 1 - tid], a.c.num_cold);
      if (cp < 0) err |= BARQ_KV_ERRBIT_BAD_INDEX;
      s_cold[tid] = cp;
    }
    __syncthreads();
    for (int q = 0; q < avail; ++q) {
      if (q > 0) pg.load(p, s_pages[q], C);
      const int cp = s_cold[q];
      if (cp >= 0) quantise_regs<KIND, NV>(a, pg, cp, s_red, s_kexp);  // uniform
      __syncthreads();  // s_red / s_kexp reused by the next block
    }
    // Every thread has read every quantised hot page: map the cold pages, push the hot pages.
    const int done = tid < avail && s_cold[tid] >= 0;
    int n_done = 0;
    const int pos = block_exclusive_scan(done, lds_scan, &n_done);
    if (n_done > 0) {  // uniform
      if (tid == 0) s_slot = atomicAdd(&p.ctrl[BARQ_KV_CTRL_FREE_TOP], n_done);
      __syncthreads();
      if (done) {
        row[s_blocks[tid]] = BARQ_KV_COLD_ENTRY(s_cold[tid]);
        const int slot = s_slot + pos;
        if (slot < p.num_pages) p.free_pages[slot] = s_pages[tid];
        else err |= BARQ_KV_ERRBIT_BAD_INDEX;
      }
    }
    __syncthreads();  // s_blocks / s_pages / s_cold reused by the next round
  }
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// ---------------------------------------------------------------------------------------------
// Gather with dequantisation: tile = (row, block, K or V); a tile's block is hot, cold or
// unmapped for all its positions, so the branch is uniform.  Vectors of VE elements along
// head_dim; output [B, H, S, D] with element strides.
// ---------------------------------------------------------------------------------------------

struct GatherArgs {
  barq_kv_pool p;
  ColdPtrs c;
  char* out[2];
  int64_t osb, osh, oss;  // elements
  int32_t batch;
  int32_t seq_out;
  int32_t nblk;           // output blocks per row
  int32_t from_device;
  FastDiv div_head;       // page_size * head_dim / VE vectors per head
  FastDiv div_dv;         // head_dim / VE
  FastDiv div_nblk;
};

template <int BYTES>
struct Raw;
template <>
struct Raw<16> { using T = uint32_t __attribute__((ext_vector_type(4))); };
template <>
struct Raw<8> { using T = uint32_t __attribute__((ext_vector_type(2))); };
template <>
struct Raw<4> { using T = uint32_t; };
template <>
struct Raw<2> { using T = uint16_t; };
template <>
struct Raw<1> { using T = uint8_t; };

template <int KIND, int VE>
struct Vec {
  using E = Elem<KIND>;
  using Bits = typename E::Bits;
  static constexpr int kBytes = VE * (int)sizeof(Bits);
  using Out = typename Raw<kBytes>::T;
  using Codes = typename Raw<VE>::T;
  union OutU {
    Out v;
    Bits e[VE];
  };
  union CodeU {
    Codes v;
    uint8_t b[VE];
  };
};

// Hardware decode of 8 codes (words w0, w1) with their 8 scale bytes (sk0, sk1): gfx950's OCP
// E4M3 conversion (exact for every finite code) times 2^(s - 127), exact in fp32 while the scale
// bytes stay in [64, 191], rounded to the output type as from_float does.  hw_decodable tells
// when it applies: NaN codes (the hardware drops their sign) and other scales take
// dequant_vec's other paths.
__device__ __forceinline__ bool hw_decodable(uint32_t w0, uint32_t w1, uint32_t sk0, uint32_t sk1) {
  const uint32_t mid = ((sk0 >> 1) ^ sk0) & ((sk1 >> 1) ^ sk1) & 0x40404040u;
  const uint32_t n0 = (w0 & 0x7F7F7F7Fu) ^ 0x7F7F7F7Fu, n1 = (w1 & 0x7F7F7F7Fu) ^ 0x7F7F7F7Fu;
  const uint32_t nan = (((n0 - 0x01010101u) & ~n0) | ((n1 - 0x01010101u) & ~n1)) & 0x80808080u;
  return mid == 0x40404040u && nan == 0;
}

// gfx950's scaled conversion: the two E4M3 codes of half HI of w times the fp32 scale s, rounded
// once to bf16.  Checked on the GPU for every code pair and every scale byte 1 .. 254 (s = 2^(b -
// 127)): identical to rounding the exact product, signed zeros included.
template <bool HI>
__device__ __forceinline__ uint32_t cvt2_bf16(uint32_t w, float s) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, s, HI));
}
__device__ __forceinline__ float e8m0_scale(uint32_t b) { return __uint_as_float(b << 23); }

template <int KIND>
__device__ __forceinline__ typename Vec<KIND, 8>::Out hw_decode(uint32_t w0, uint32_t w1, uint32_t sk0, uint32_t sk1) {
  using V = Vec<KIND, 8>;
  using E = Elem<KIND>;
  using Bits = typename E::Bits;
  typename V::OutU val;
  if constexpr (KIND == BARQ_KV_BF16) {
    // two conversions per pair of codes, one with each code's scale, and a half of each kept
    uint32_t r[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const uint32_t w = j ? w1 : w0, sw = j ? sk1 : sk0;
      const uint32_t a0 = cvt2_bf16<false>(w, e8m0_scale(sw & 0xFFu));
      const uint32_t b0 = cvt2_bf16<false>(w, e8m0_scale((sw >> 8) & 0xFFu));
      const uint32_t a1 = cvt2_bf16<true>(w, e8m0_scale((sw >> 16) & 0xFFu));
      const uint32_t b1 = cvt2_bf16<true>(w, e8m0_scale(sw >> 24));
      r[2 * j] = (a0 & 0xFFFFu) | (b0 & 0xFFFF0000u);
      r[2 * j + 1] = (a1 & 0xFFFFu) | (b1 & 0xFFFF0000u);
    }
    return typename V::Out{r[0], r[1], r[2], r[3]};
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const uint32_t w = j ? w1 : w0, sw = j ? sk1 : sk0;
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    const float f[4] = {lo[0] * __uint_as_float((sw & 0xFFu) << 23),
                        lo[1] * __uint_as_float(((sw >> 8) & 0xFFu) << 23),
                        hi[0] * __uint_as_float(((sw >> 16) & 0xFFu) << 23),
                        hi[1] * __uint_as_float((sw >> 24) << 23)};
    // The hardware reads code 0x80 as +0: every code's sign bit goes back on its value.
    if constexpr (KIND == BARQ_KV_BF16) {  // exact values: the top halves
      const uint32_t p0 = __builtin_amdgcn_perm(__float_as_uint(f[1]), __float_as_uint(f[0]), 0x07060302u) |
                          ((w << 8) & 0x8000u) | ((w << 16) & 0x80000000u);
      const uint32_t p1 = __builtin_amdgcn_perm(__float_as_uint(f[3]), __float_as_uint(f[2]), 0x07060302u) |
                          ((w >> 8) & 0x8000u) | (w & 0x80000000u);
      val.e[4 * j] = (Bits)p0;
      val.e[4 * j + 1] = (Bits)(p0 >> 16);
      val.e[4 * j + 2] = (Bits)p1;
      val.e[4 * j + 3] = (Bits)(p1 >> 16);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        val.e[4 * j + e] = (Bits)(E::from_float(f[e]) | (((w >> (8 * e + 7)) & 1u) << 15));
    }
  }
  return val.v;
}

// hw_decode for one scale byte over all 8 codes (a value vector: one scale per position and head).
template <int KIND>
__device__ __forceinline__ typename Vec<KIND, 8>::Out hw_decode_one(uint32_t w0, uint32_t w1, uint32_t sb) {
  if constexpr (KIND == BARQ_KV_BF16) {
    const float s = e8m0_scale(sb);
    return typename Vec<KIND, 8>::Out{cvt2_bf16<false>(w0, s), cvt2_bf16<true>(w0, s), cvt2_bf16<false>(w1, s),
                                      cvt2_bf16<true>(w1, s)};
  } else {
    return hw_decode<KIND>(w0, w1, sb * 0x01010101u, sb * 0x01010101u);
  }
}

// VE elements from their E4M3 codes and scales: keys with VE per-channel scale bytes (ksc),
// values with one per-token scale byte (vsc).  Exact: code * 2^(s - 127) rounded once to the
// element type.
template <int KIND, int VE>
__device__ __forceinline__ typename Vec<KIND, VE>::Out dequant_vec(typename Vec<KIND, VE>::CodeU codes,
                                                                  typename Vec<KIND, VE>::CodeU ksc, uint32_t vsc,
                                                                  int kv) {
  using V = Vec<KIND, VE>;
  using E = Elem<KIND>;
  typename V::OutU val;
  if constexpr (VE == 8 && KIND != BARQ_KV_FP32) {
    const uint32_t w0 = codes.v.x, w1 = codes.v.y;
    const uint32_t sk0 = kv == 0 ? ksc.v.x : vsc * 0x01010101u;
    const uint32_t sk1 = kv == 0 ? ksc.v.y : vsc * 0x01010101u;
    if (hw_decodable(w0, w1, sk0, sk1)) return hw_decode<KIND>(w0, w1, sk0, sk1);
    uint32_t s0, s1, s2, s3;  // scale pairs, spread like the code pairs
    bool fast = codes_normal(w0) && codes_normal(w1);
    if (kv == 0) {
#pragma unroll
      for (int e = 0; e < VE; ++e) fast = fast && scale_fast<KIND>(ksc.b[e]);
      s0 = spread_lo(ksc.v.x);
      s1 = spread_hi(ksc.v.x);
      s2 = spread_lo(ksc.v.y);
      s3 = spread_hi(ksc.v.y);
    } else {
      fast = fast && scale_fast<KIND>(vsc);
      s0 = s1 = s2 = s3 = vsc | (vsc << 16);
    }
    if (fast) {
      uint32_t r[4] = {fast_pair<KIND>(spread_lo(w0), s0), fast_pair<KIND>(spread_hi(w0), s1),
                       fast_pair<KIND>(spread_lo(w1), s2), fast_pair<KIND>(spread_hi(w1), s3)};
      return *(typename V::Out*)r;
    }
  }
  if (kv == 0) {
#pragma unroll
    for (int e = 0; e < VE; ++e) val.e[e] = E::from_float(ldexpf(e4m3_decode(codes.b[e]), (int)ksc.b[e] - 127));
  } else {
#pragma unroll
    for (int e = 0; e < VE; ++e) val.e[e] = E::from_float(ldexpf(e4m3_decode(codes.b[e]), (int)vsc - 127));
  }
  return val.v;
}

template <int KIND, int VE>
__global__ void __launch_bounds__(kGatherThreads) gather_cold_kernel(const GatherArgs a) {
  using V = Vec<KIND, VE>;
  using E = Elem<KIND>;
  using Bits = typename E::Bits;
  __shared__ int s_seq;
  const barq_kv_pool& p = a.p;
  const int kv = blockIdx.x & 1;
  const int bj = blockIdx.x >> 1;
  const int b = (int)a.div_nblk.div((uint32_t)bj);
  const int j = bj - b * a.nblk;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim;
  const int pos0 = j * P;
  // The row's mark and the block's entry are read together with the lengths (one round trip).
  const int hw = p.high_water[b];
  const int stored = p.block_table[(int64_t)b * p.max_blocks + j];
  // The extent (longest row) matters only to a block reaching past its row's length: the others
  // hold data at every position and skip the batch-wide read.
  const bool need_extent = a.from_device && pos0 + P > p.seq_lens[b];
  if (need_extent) {  // uniform
    if (threadIdx.x < kWave) {
      int m = 0;
      for (int i = threadIdx.x; i < a.batch; i += kWave) m = max(m, p.seq_lens[i]);
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, kWave));
      if (threadIdx.x == 0) s_seq = min(m, a.seq_out);
    }
    __syncthreads();
  }
  const int S = need_extent ? s_seq : a.seq_out;
  if (pos0 >= S) return;  // uniform
  const int entry = pos0 < hw ? stored : -1;
  const int hot = checked_id(entry, p.num_pages);
  const int cold = entry <= -2 ? checked_id(-2 - entry, a.c.num_cold) : -1;
  if (entry <= -2 && cold < 0 && threadIdx.x == 0) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], BARQ_KV_ERRBIT_BAD_INDEX);
  const int dv_n = (int)a.div_dv.d;
  const int nvec = H * P * dv_n;
  Bits* out = (Bits*)a.out[kv] + (int64_t)b * a.osb;
  const int live = min(S, hw) - pos0;  // positions of this block with data
  const int end = min(S - pos0, P);    // positions of this block in the output
  const int slot = hot >= 0 ? hot : cold;
  // Every load of a round is issued before any value is used (one round trip per round).
  for (int v0 = threadIdx.x; v0 < nvec; v0 += kGatherThreads * kUnroll) {
    typename V::OutU val[kUnroll];
    int64_t at[kUnroll], el[kUnroll];
    int tok[kUnroll], head[kUnroll], col[kUnroll];
    bool in[kUnroll], has[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int v = v0 + u * kGatherThreads;
      const int h = (int)a.div_head.div((uint32_t)v);
      const int rem = v - h * (int)a.div_head.d;
      const int t = (int)a.div_dv.div((uint32_t)rem);
      const int dv = rem - t * dv_n;
      in[u] = v < nvec && t < end;
      has[u] = in[u] && t < live && slot >= 0;
      at[u] = (int64_t)h * a.osh + (int64_t)(pos0 + t) * a.oss + (int64_t)dv * VE;
      el[u] = (((int64_t)slot * P + t) * H + h) * D + (int64_t)dv * VE;
      tok[u] = t;
      head[u] = h;
      col[u] = dv * VE;
      val[u].v = typename V::Out(0);
    }
    if (hot >= 0) {  // uniform
      const char* base = kv ? (const char*)p.value_pages : (const char*)p.key_pages;
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        if (has[u]) val[u].v = __builtin_nontemporal_load((const typename V::Out*)(base + el[u] * (int64_t)sizeof(Bits)));
    } else if (cold >= 0) {  // uniform
      typename V::CodeU codes[kUnroll], ksc[kUnroll];
      uint32_t vsc[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        codes[u].v = typename V::Codes(0);
        ksc[u].v = typename V::Codes(0);
        vsc[u] = 0;
        if (!has[u]) continue;
        codes[u].v = __builtin_nontemporal_load((const typename V::Codes*)(a.c.codes[kv] + el[u]));
        if (kv == 0)
          ksc[u].v = *(const typename V::Codes*)(a.c.key_scales + ((int64_t)cold * H + head[u]) * D + col[u]);
        else
          vsc[u] = a.c.value_scales[((int64_t)cold * P + tok[u]) * H + head[u]];
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u)
        if (has[u]) val[u].v = dequant_vec<KIND, VE>(codes[u], ksc[u], vsc[u], kv);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u)
      if (in[u]) __builtin_nontemporal_store(val[u].v, (typename V::Out*)(out + at[u]));
  }
}

// dequant_vec's exact path for 8 codes (words w0, w1) and their scale bytes (sk0, sk1), one
// element at a time: the rare path of the lanes kernels, holding one element's registers.
template <int KIND>
__device__ __forceinline__ typename Vec<KIND, 8>::Out exact8(uint32_t w0, uint32_t w1, uint32_t sk0, uint32_t sk1) {
  uint32_t r0 = 0, r1 = 0, r2 = 0, r3 = 0;
#pragma unroll 1
  for (int e = 0; e < 8; ++e) {
    const int sh = 8 * (e & 3);
    const uint32_t code = ((e < 4 ? w0 : w1) >> sh) & 0xFFu;
    const int sc = (int)(((e < 4 ? sk0 : sk1) >> sh) & 0xFFu);
    const uint32_t bits = (uint32_t)Elem<KIND>::from_float(ldexpf(e4m3_decode(code), sc - 127)) << (16 * (e & 1));
    const int word = e >> 1;
    r0 |= word == 0 ? bits : 0u;
    r1 |= word == 1 ? bits : 0u;
    r2 |= word == 2 ? bits : 0u;
    r3 |= word == 3 ? bits : 0u;
  }
  return typename Vec<KIND, 8>::Out{r0, r1, r2, r3};
}

// One wave's round of a cold tile in the lanes kernels (VALUES: the V page, whose scales are
// per position and head; else K, per-channel scales ksc): positions t0 .. t0 + 8 / LPP - 1 of
// the page, decoded below `live`, zeros up to `end`; the lane's columns col[c] (element offsets
// in a token row) go to ocol[c] of the output rows at o.  The round's codes and scales load
// together and unconditionally (positions clamped into the page): a load under a condition
// leaves a phi of zero and the loaded value, into whose block the compiler moves the scale
// arithmetic, waiting there for each load before the next is issued.  A vector decodes on the
// hardware path when every lane's does (scales in [64, 191], no NaN code: the usual case), else
// element by element; with dequant_vec inlined for the whole round the kernels held 4 waves per
// SIMD instead of 5.  `spaced` (uniform): each store waits for the previous one, one store in
// flight per wave.
template <int KIND, int LPP, bool VALUES>
__device__ __forceinline__ void cold_round(const GatherArgs& a, int cold, int t0, int live, int end, int lane,
                                           const int (&col)[LPP], const int64_t (&ocol)[LPP],
                                           const typename Vec<KIND, 8>::CodeU (&ksc)[LPP],
                                           typename Elem<KIND>::Bits* o, bool spaced) {
  using V = Vec<KIND, 8>;
  constexpr int kNPos = 8 / LPP;
  const barq_kv_pool& p = a.p;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim;
  const int HD = H * D;
  const int dvn = D / 8;
  const uint8_t* codes = a.c.codes[VALUES ? 1 : 0] + (int64_t)cold * P * HD;
  const uint8_t* vscales = a.c.value_scales + (int64_t)cold * P * H;
  typename V::CodeU cv[kNPos][LPP];
  uint32_t vsc[kNPos][LPP];
#pragma unroll
  for (int i = 0; i < kNPos; ++i) {
    const int t = min(t0 + i, P - 1);
#pragma unroll
    for (int c = 0; c < LPP; ++c) {
      cv[i][c].v = __builtin_nontemporal_load((const typename V::Codes*)(codes + (int64_t)t * HD + col[c]));
      vsc[i][c] = VALUES ? vscales[t * H + (c * kWave + lane) / dvn] : 0u;
    }
  }
#pragma unroll
  for (int i = 0; i < kNPos; ++i)
#pragma unroll
    for (int c = 0; c < LPP; ++c) {
      if (t0 + i >= end) continue;
      const uint32_t w0 = cv[i][c].v.x, w1 = cv[i][c].v.y;
      const uint32_t sk0 = VALUES ? vsc[i][c] * 0x01010101u : ksc[c].v.x;
      const uint32_t sk1 = VALUES ? vsc[i][c] * 0x01010101u : ksc[c].v.y;
      const bool dead = t0 + i >= live;
      typename V::Out v;
      if (__builtin_amdgcn_ballot_w64(!(dead || hw_decodable(w0, w1, sk0, sk1))) == 0) {  // uniform
        if constexpr (VALUES)
          v = hw_decode_one<KIND>(w0, w1, vsc[i][c]);
        else
          v = hw_decode<KIND>(w0, w1, sk0, sk1);
      } else
        v = exact8<KIND>(w0, w1, sk0, sk1);
      if (dead) v = typename V::Out(0);
      if (spaced) wait_vm<0>();
      __builtin_nontemporal_store(v, (typename V::Out*)(o + (int64_t)i * a.oss + ocol[c]));
    }
}

// The gather for 8-element vectors (2-byte elements) when a token's kv_heads * head_dim
// elements are 64 * LPP vectors: a wave moves whole positions, lane l taking vectors l, l + 64,
// ... of each, so a lane's columns -- and its key scales -- are fixed for the tile and only the
// position varies (wave-uniform).  Each wave holds 8 vectors per lane in flight (8 / LPP
// positions a round); per-channel key scales are read once per tile.
template <int KIND, int LPP>
__global__ void __launch_bounds__(kGatherThreads) gather_cold_lanes_kernel(const GatherArgs a) {
  using V = Vec<KIND, 8>;
  using E = Elem<KIND>;
  using Bits = typename E::Bits;
  constexpr int kNPos = 8 / LPP;  // positions a wave moves per round
  constexpr int kWavesPerTile = kGatherThreads / kWave;
  __shared__ int s_seq;
  const barq_kv_pool& p = a.p;
  const int kv = blockIdx.x & 1;
  const int bj = blockIdx.x >> 1;
  const int b = (int)a.div_nblk.div((uint32_t)bj);
  const int j = bj - b * a.nblk;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim;
  const int pos0 = j * P;
  const int hw = p.high_water[b];
  const int stored = p.block_table[(int64_t)b * p.max_blocks + j];
  // The extent (longest row) matters only to a block reaching past its row's length: the others
  // hold data at every position and skip the batch-wide read.
  const bool need_extent = a.from_device && pos0 + P > p.seq_lens[b];
  if (need_extent) {  // uniform
    if (threadIdx.x < kWave) {
      int m = 0;
      for (int i = threadIdx.x; i < a.batch; i += kWave) m = max(m, p.seq_lens[i]);
#pragma unroll
      for (int o = kWave / 2; o > 0; o >>= 1) m = max(m, __shfl_xor(m, o, kWave));
      if (threadIdx.x == 0) s_seq = min(m, a.seq_out);
    }
    __syncthreads();
  }
  const int S = need_extent ? s_seq : a.seq_out;
  if (pos0 >= S) return;  // uniform
  const int entry = pos0 < hw ? stored : -1;
  const int hot = checked_id(entry, p.num_pages);
  const int cold = entry <= -2 ? checked_id(-2 - entry, a.c.num_cold) : -1;
  if (entry <= -2 && cold < 0 && threadIdx.x == 0) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], BARQ_KV_ERRBIT_BAD_INDEX);
  const int live = min(S, hw) - pos0;
  const int end = min(S - pos0, P);
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int HD = H * D;
  const int dvn = D / 8;
  // this lane's columns: element offsets within a token row and within an output position
  int col[LPP];
  int64_t ocol[LPP];
#pragma unroll
  for (int c = 0; c < LPP; ++c) {
    const int vi = c * kWave + lane;
    const int h = vi / dvn;
    col[c] = vi * 8;
    ocol[c] = (int64_t)h * a.osh + (int64_t)(vi - h * dvn) * 8;
  }
  Bits* out = (Bits*)a.out[kv] + (int64_t)b * a.osb + (int64_t)pos0 * a.oss;
  typename V::CodeU ksc[LPP];
  if (cold >= 0 && kv == 0) {
#pragma unroll
    for (int c = 0; c < LPP; ++c) ksc[c].v = *(const typename V::Codes*)(a.c.key_scales + (int64_t)cold * HD + col[c]);
  }
  for (int t0 = wave * kNPos; t0 < end; t0 += kWavesPerTile * kNPos) {
    Bits* o = out + (int64_t)t0 * a.oss;
    if (hot >= 0) {  // uniform: a copy, every load of the round in flight before the stores
      const char* base = (kv ? (const char*)p.value_pages : (const char*)p.key_pages) +
                         ((int64_t)hot * P + t0) * HD * (int64_t)sizeof(Bits);
      typename V::OutU val[kNPos][LPP];
#pragma unroll
      for (int i = 0; i < kNPos; ++i)
#pragma unroll
        for (int c = 0; c < LPP; ++c) {
          val[i][c].v = typename V::Out(0);
          if (t0 + i < live)
            val[i][c].v = __builtin_nontemporal_load(
                (const typename V::Out*)(base + ((int64_t)i * HD + col[c]) * (int64_t)sizeof(Bits)));
        }
#pragma unroll
      for (int i = 0; i < kNPos; ++i)
#pragma unroll
        for (int c = 0; c < LPP; ++c)
          if (t0 + i < end) __builtin_nontemporal_store(val[i][c].v, (typename V::Out*)(o + (int64_t)i * a.oss + ocol[c]));
    } else if (cold >= 0) {  // uniform
      if (kv)
        cold_round<KIND, LPP, true>(a, cold, t0, live, end, lane, col, ocol, ksc, o, false);
      else
        cold_round<KIND, LPP, false>(a, cold, t0, live, end, lane, col, ocol, ksc, o, false);
    } else {
#pragma unroll
      for (int i = 0; i < kNPos; ++i)
#pragma unroll
        for (int c = 0; c < LPP; ++c)
          if (t0 + i < end) __builtin_nontemporal_store(typename V::Out(0), (typename V::Out*)(o + (int64_t)i * a.oss + ocol[c]));
    }
  }
}

// The dequantising update in one launch, for tokens <= window (the blocks that leave the window
// were quantised just before, from the lengths the rows are about to reach): the tiles of
// gather_cold_lanes_kernel, whose rows also receive `tokens` new positions.  Every tile reads
// the launch's starting state -- the row's length and mark, its block's entry, the output extent
// (longest row + tokens), and for a block the append maps first the page its rank takes from the
// stack -- then arrives; the last tile to arrive commits the append (barq_commit, as the stream
// kernels do).  New positions are taken from the input, written to the output and to their hot
// page; a tile holding none runs gather_cold_lanes_kernel's copy or decode unchanged.
struct UpdateArgs {
  GatherArgs g;
  const char* in[2];      // key, value states
  int64_t isb, ish, ist;  // input strides, elements
  int32_t tokens;
  int32_t nsub;           // arrival sub-counters in use
  int32_t spaced;         // every tile resident at once: one store in flight per wave (3 % faster
                          // at C2); launches of several rounds keep their stores back to back
  FastDiv div_page;
};

template <int KIND, int LPP>
__global__ void __launch_bounds__(kGatherThreads) __attribute__((amdgpu_waves_per_eu(LPP <= 2 ? 5 : 3))) update_cold_lanes_kernel(const UpdateArgs u) {
  using V = Vec<KIND, 8>;
  using E = Elem<KIND>;
  using Bits = typename E::Bits;
  constexpr int kNPos = 8 / LPP;  // positions a wave moves per round
  constexpr int kWavesPerTile = kGatherThreads / kWave;
  const GatherArgs& a = u.g;
  const barq_kv_pool& p = a.p;
  const int kv = blockIdx.x & 1;
  const int bj = blockIdx.x >> 1;
  const int b = (int)a.div_nblk.div((uint32_t)bj);
  const int j = bj - b * a.nblk;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim;
  const int T = u.tokens;
  const int mb = (int)p.max_blocks;
  const int pos0 = j * P;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);

  // The launch's starting state (batch <= 64: one row per lane).
  const int len = p.seq_lens[b];
  const int hw = p.high_water[b];
  const int stored = p.block_table[(int64_t)b * mb + j];
  // The extent (longest row + tokens) matters only to a block reaching past its row's new end:
  // the others hold data at every position and skip the batch-wide read (every tile reading the
  // same lengths serialises on one L2 channel).
  int S = a.seq_out;
  if (a.from_device && pos0 + P > len + T)
    S = min(barq_commit::wave_max(lane < a.batch ? p.seq_lens[lane] + T : 0), a.seq_out);
  const barq_commit::NewBlocks nb = barq_commit::new_blocks(len, hw, T, mb, u.div_page);
  const bool fresh_block = j >= nb.first && j < nb.first + nb.count;
  int newpage = -1;
  if (fresh_block) {
    const int top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
    const int base = barq_commit::wave_sum(
        lane < b ? barq_commit::new_blocks(p.seq_lens[lane], p.high_water[lane], T, mb, u.div_page).count : 0);
    const int idx = top - 1 - (base + j - nb.first);
    newpage = idx >= 0 ? checked_id(p.free_pages[idx], p.num_pages) : -1;
  }
  __builtin_amdgcn_s_waitcnt(0);  // every wave holds its metadata before the tile arrives
  __syncthreads();
  if (wave == 0) barq_commit::arrive_and_commit(p, u.nsub, a.batch, T, a.seq_out, u.div_page);
  if (pos0 >= S) return;  // uniform

  const bool old_block = pos0 < hw;  // mapped before this append
  const int entry = old_block ? stored : -1;
  const int hot = old_block ? checked_id(entry, p.num_pages) : newpage;
  const int cold = entry <= -2 ? checked_id(-2 - entry, a.c.num_cold) : -1;
  if (entry <= -2 && cold < 0 && threadIdx.x == 0) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], BARQ_KV_ERRBIT_BAD_INDEX);
  const int live = min(S, hw) - pos0;  // old data: positions below the mark
  const int end = min(S - pos0, P);
  const int f_lo = len - pos0;         // new positions of the tile: [f_lo, f_lo + T) within [0, end)
  const bool fresh_tile = f_lo < end && f_lo + T > 0;
  const int HD = H * D;
  const int dvn = D / 8;
  int col[LPP];
  int64_t ocol[LPP], icol[LPP];
#pragma unroll
  for (int c = 0; c < LPP; ++c) {
    const int vi = c * kWave + lane;
    const int h = vi / dvn;
    col[c] = vi * 8;
    ocol[c] = (int64_t)h * a.osh + (int64_t)(vi - h * dvn) * 8;
    icol[c] = (int64_t)h * u.ish + (int64_t)(vi - h * dvn) * 8;
  }
  Bits* out = (Bits*)a.out[kv] + (int64_t)b * a.osb + (int64_t)pos0 * a.oss;
  char* page_base = hot >= 0 ? (kv ? (char*)p.value_pages : (char*)p.key_pages) +
                                   (int64_t)hot * P * HD * (int64_t)sizeof(Bits)
                             : nullptr;
  if (fresh_tile) {
    // New positions from the input (to the output and their page), old ones from the hot page.
    const Bits* in = (const Bits*)u.in[kv] + (int64_t)b * u.isb;
    if (cold >= 0 && threadIdx.x == 0) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], BARQ_KV_ERRBIT_BAD_INDEX);
    for (int t0 = wave * kNPos; t0 < end; t0 += kWavesPerTile * kNPos) {
      typename V::OutU val[kNPos][LPP];
#pragma unroll
      for (int i = 0; i < kNPos; ++i) {
        const int t = t0 + i;
        const bool fresh = (unsigned)(t - f_lo) < (unsigned)T;
#pragma unroll
        for (int c = 0; c < LPP; ++c) {
          val[i][c].v = typename V::Out(0);
          if (t < end && fresh)
            val[i][c].v = __builtin_nontemporal_load(
                (const typename V::Out*)(in + (int64_t)(t - f_lo) * u.ist + icol[c]));
          else if (t < live && hot >= 0)
            val[i][c].v = __builtin_nontemporal_load(
                (const typename V::Out*)(page_base + ((int64_t)t * HD + col[c]) * (int64_t)sizeof(Bits)));
        }
      }
#pragma unroll
      for (int i = 0; i < kNPos; ++i) {
        const int t = t0 + i;
        if (t >= end) continue;
        const bool fresh = (unsigned)(t - f_lo) < (unsigned)T;
#pragma unroll
        for (int c = 0; c < LPP; ++c) {
          __builtin_nontemporal_store(val[i][c].v, (typename V::Out*)(out + (int64_t)t * a.oss + ocol[c]));
          if (fresh && hot >= 0)
            *(typename V::Out*)(page_base + ((int64_t)t * HD + col[c]) * (int64_t)sizeof(Bits)) = val[i][c].v;
        }
      }
    }
    return;
  }
  typename V::CodeU ksc[LPP];
  if (cold >= 0 && kv == 0) {
#pragma unroll
    for (int c = 0; c < LPP; ++c) ksc[c].v = *(const typename V::Codes*)(a.c.key_scales + (int64_t)cold * HD + col[c]);
  }
  for (int t0 = wave * kNPos; t0 < end; t0 += kWavesPerTile * kNPos) {
    Bits* o = out + (int64_t)t0 * a.oss;
    if (hot >= 0) {  // uniform: a copy, every load of the round in flight before the stores
      const char* base = page_base + (int64_t)t0 * HD * (int64_t)sizeof(Bits);
      typename V::OutU val[kNPos][LPP];
#pragma unroll
      for (int i = 0; i < kNPos; ++i)
#pragma unroll
        for (int c = 0; c < LPP; ++c) {
          val[i][c].v = typename V::Out(0);
          if (t0 + i < live)
            val[i][c].v = __builtin_nontemporal_load(
                (const typename V::Out*)(base + ((int64_t)i * HD + col[c]) * (int64_t)sizeof(Bits)));
        }
#pragma unroll
      for (int i = 0; i < kNPos; ++i)
#pragma unroll
        for (int c = 0; c < LPP; ++c)
          if (t0 + i < end) {
            if (u.spaced) wait_vm<0>();
            __builtin_nontemporal_store(val[i][c].v, (typename V::Out*)(o + (int64_t)i * a.oss + ocol[c]));
          }
    } else if (cold >= 0) {  // uniform
      if (kv)
        cold_round<KIND, LPP, true>(a, cold, t0, live, end, lane, col, ocol, ksc, o, u.spaced);
      else
        cold_round<KIND, LPP, false>(a, cold, t0, live, end, lane, col, ocol, ksc, o, u.spaced);
    } else {
#pragma unroll
      for (int i = 0; i < kNPos; ++i)
#pragma unroll
        for (int c = 0; c < LPP; ++c)
          if (t0 + i < end) __builtin_nontemporal_store(typename V::Out(0), (typename V::Out*)(o + (int64_t)i * a.oss + ocol[c]));
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Row release with a cold store: one workgroup, a row at a time; hot pages (shares-aware) go back
// to free_pages, cold pages to free_cold, each in (row, block) order.
// ---------------------------------------------------------------------------------------------

struct FreeArgs {
  barq_kv_pool p;
  ColdPtrs c;
  const int32_t* rows;
  int32_t n;
  FastDiv div_page;
};

__global__ void __launch_bounds__(kThreads) free_rows_cold_kernel(const FreeArgs a) {
  __shared__ int lds_scan[kWaves];
  const barq_kv_pool& p = a.p;
  const int hot_top = p.ctrl[BARQ_KV_CTRL_FREE_TOP];
  const int cold_top = p.ctrl[BARQ_KV_CTRL_COLD_TOP];
  const int mb = (int)p.max_blocks;
  int hot_pushed = 0, cold_pushed = 0, err = 0;
  for (int i = 0; i < a.n; ++i) {
    const int r = a.rows[i];
    if (r < 0 || r >= (int)p.max_batch) {
      err |= BARQ_KV_ERRBIT_BAD_INDEX;
      continue;
    }
    const int cnt = min(ceil_div_fd(p.high_water[r], a.div_page), mb);
    int32_t* row = p.block_table + (int64_t)r * mb;
    for (int j0 = 0; j0 < cnt; j0 += kThreads) {
      const int j = j0 + (int)threadIdx.x;
      int hot = -1, cold = -1;
      if (j < cnt) {
        const int e = row[j];
        hot = checked_id(e, p.num_pages);
        if (e <= -2) cold = checked_id(-2 - e, a.c.num_cold);
        if (hot >= 0 && p.page_shares && atomicSub(&p.page_shares[hot], 1) != 0) hot = -1;
        else if (hot >= 0 && p.page_shares) p.page_shares[hot] = 0;
        if (cold >= 0 && a.c.shares && atomicSub(&a.c.shares[cold], 1) != 0) cold = -1;
        else if (cold >= 0 && a.c.shares) a.c.shares[cold] = 0;
        row[j] = -1;
      }
      int hot_n = 0, cold_n = 0;
      const int hk = block_exclusive_scan(hot >= 0, lds_scan, &hot_n);
      const int ck = block_exclusive_scan(cold >= 0, lds_scan, &cold_n);
      if (hot >= 0) {
        const int64_t slot = (int64_t)hot_top + hot_pushed + hk;
        if (slot < p.num_pages) p.free_pages[slot] = hot;
        else err |= BARQ_KV_ERRBIT_BAD_INDEX;
      }
      if (cold >= 0) {
        const int64_t slot = (int64_t)cold_top + cold_pushed + ck;
        if (slot < a.c.num_cold) a.c.free_cold[slot] = cold;
        else err |= BARQ_KV_ERRBIT_BAD_INDEX;
      }
      hot_pushed += hot_n;
      cold_pushed += cold_n;
    }
    __syncthreads();  // every thread has read the row's mark before it is cleared
    if (threadIdx.x == 0) {
      p.seq_lens[r] = 0;
      p.high_water[r] = 0;
    }
  }
  if (threadIdx.x == 0) {
    p.ctrl[BARQ_KV_CTRL_FREE_TOP] = (int)std::min<int64_t>((int64_t)hot_top + hot_pushed, p.num_pages);
    p.ctrl[BARQ_KV_CTRL_COLD_TOP] = (int)std::min<int64_t>((int64_t)cold_top + cold_pushed, a.c.num_cold);
  }
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

__global__ void cold_reset_kernel(ColdPtrs c, int32_t* ctrl) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < c.num_cold) c.free_cold[i] = (int32_t)(c.num_cold - 1 - i);
  if (i < c.num_cold && c.shares) c.shares[i] = 0;
  if (i == 0) ctrl[BARQ_KV_CTRL_COLD_TOP] = (int32_t)c.num_cold;
}

// ---------------------------------------------------------------------------------------------
// Crop with a cold store: workgroup per row.  The row's quantised blocks from the one holding its
// new length on are re-opened: a page popped from free_pages receives the block's dequantised K
// and V (code * 2^e rounded to the element type, as the gather reads it), the block maps it, and
// the cold page loses the reference.
// ---------------------------------------------------------------------------------------------

struct CropArgs {
  barq_kv_pool p;
  ColdPtrs c;
  int32_t batch;
  int32_t max_length;
  FastDiv div_page;
};

template <int KIND>
__global__ void __launch_bounds__(kThreads) crop_cold_kernel(const CropArgs a) {
  using E = Elem<KIND>;
  using Bits = typename E::Bits;
  __shared__ int lds_scan[kWaves];
  __shared__ int s_block[kThreads];  // the chunk's re-opened blocks ...
  __shared__ int s_hot[kThreads];    // ... and the pages they take (-1: none left)
  __shared__ int s_base;
  const barq_kv_pool& p = a.p;
  const int r = blockIdx.x;
  const int mb = (int)p.max_blocks;
  const int P = (int)p.page_size, H = (int)p.kv_heads, D = (int)p.head_dim;
  const int HD = H * D;
  const int len = min(p.seq_lens[r], a.max_length);
  const int first = (int)a.div_page.div((uint32_t)len);
  const int nb = min(ceil_div_fd(p.high_water[r], a.div_page), mb);
  int32_t* row = p.block_table + (int64_t)r * mb;
  int err = 0;
  for (int j0 = first; j0 < nb; j0 += kThreads) {
    const int j = j0 + (int)threadIdx.x;
    int c = -1;
    if (j < nb) {
      const int e = row[j];
      if (e <= -2) c = checked_id(-2 - e, a.c.num_cold);
    }
    int count = 0;
    const int k = block_exclusive_scan(c >= 0, lds_scan, &count);
    if (threadIdx.x == 0 && count > 0) {
      const int before = atomicSub(&p.ctrl[BARQ_KV_CTRL_FREE_TOP], count);
      const int got = max(0, min(before, count));
      if (got < count) {
        atomicAdd(&p.ctrl[BARQ_KV_CTRL_FREE_TOP], count - got);
        err |= BARQ_KV_ERRBIT_POOL_EXHAUSTED;
      }
      s_base = before - got;  // pages [s_base, s_base + got) of the stack, the top one first
      s_hot[0] = got;         // read before the per-block entries below are written
    }
    __syncthreads();
    const int got = s_hot[0], base = s_base;
    __syncthreads();
    if (c >= 0) {
      s_block[k] = j;
      s_hot[k] = k < got ? checked_id(p.free_pages[base + got - 1 - k], p.num_pages) : -1;
      if (k < got && s_hot[k] < 0) err |= BARQ_KV_ERRBIT_BAD_INDEX;
    }
    __syncthreads();
    for (int q = 0; q < min(count, got); ++q) {
      const int jb = s_block[q], hp = s_hot[q];
      const int cp = -2 - row[jb];  // every thread reads the entry before thread 0 rewrites it
      __syncthreads();
      if (hp < 0) continue;  // uniform
      Bits* kp = (Bits*)p.key_pages + (int64_t)hp * P * HD;
      Bits* vp = (Bits*)p.value_pages + (int64_t)hp * P * HD;
      const uint8_t* kc = a.c.codes[0] + (int64_t)cp * P * HD;
      const uint8_t* vc = a.c.codes[1] + (int64_t)cp * P * HD;
      for (int i = threadIdx.x; i < P * HD; i += kThreads) {
        const int t = i / HD, hd = i - t * HD, h = hd / D;
        const int ek = (int)a.c.key_scales[(int64_t)cp * HD + hd] - 127;
        const int ev = (int)a.c.value_scales[((int64_t)cp * P + t) * H + h] - 127;
        kp[i] = E::from_float(ldexpf(e4m3_decode(kc[i]), ek));
        vp[i] = E::from_float(ldexpf(e4m3_decode(vc[i]), ev));
      }
      __syncthreads();  // the cold page is read in full before it can return to the stack
      if (threadIdx.x == 0) {
        row[jb] = hp;
        if (!a.c.shares || atomicSub(&a.c.shares[cp], 1) == 0) {
          if (a.c.shares) a.c.shares[cp] = 0;
          const int slot = atomicAdd(&p.ctrl[BARQ_KV_CTRL_COLD_TOP], 1);
          if (slot < a.c.num_cold) a.c.free_cold[slot] = cp;
          else err |= BARQ_KV_ERRBIT_BAD_INDEX;
        }
      }
    }
    __syncthreads();
  }
  __syncthreads();  // every thread has read the row's length before it is lowered
  if (threadIdx.x == 0 && r < a.batch) p.seq_lens[r] = len;
  if (err) atomicOr(&p.ctrl[BARQ_KV_CTRL_ERRORS], err);
}

// ---------------------------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------------------------

bool pool_ok(const barq_kv_pool* p) {
  if (!p || !p->key_pages || !p->value_pages || !p->block_table || !p->seq_lens || !p->high_water ||
      !p->free_pages || !p->ctrl)
    return false;
  if (p->num_pages < 1 || p->num_pages > kI32Max || p->max_batch < 1 || p->max_batch > kI32Max ||
      p->max_blocks < 1 || p->page_size < 1 || p->kv_heads < 1 || p->head_dim < 1)
    return false;
  if (p->max_batch * p->max_blocks > kI32Max || p->max_blocks * p->page_size > kI32Max) return false;
  return p->elem_bytes == 2 || p->elem_bytes == 4;
}

bool cold_ok(const barq_kv_pool* p, const barq_kv_cold* c) {
  if (!pool_ok(p) || !c || !c->key_codes || !c->value_codes || !c->key_scales || !c->value_scales ||
      !c->free_cold)
    return false;
  if (c->num_cold < 1 || c->num_cold > kI32Max - 2 || c->window < 0 || c->window > kI32Max) return false;
  const int64_t want = c->element_type == BARQ_KV_FP32 ? 4 : 2;
  if (c->element_type < BARQ_KV_BF16 || c->element_type > BARQ_KV_FP32 || p->elem_bytes != want) return false;
  return p->page_size * p->kv_heads <= kMaxTokenHeads && p->kv_heads * p->head_dim <= kMaxChannels;
}

ColdPtrs cold_ptrs(const barq_kv_cold* c) {
  ColdPtrs r;
  r.codes[0] = (uint8_t*)c->key_codes;
  r.codes[1] = (uint8_t*)c->value_codes;
  r.key_scales = (uint8_t*)c->key_scales;
  r.value_scales = (uint8_t*)c->value_scales;
  r.free_cold = c->free_cold;
  r.shares = c->cold_shares;
  r.num_cold = c->num_cold;
  r.window = (int32_t)c->window;
  return r;
}

int launch(const void* fn, dim3 grid, void* arg, hipStream_t stream) {
  void* args[] = {arg};
  return hipLaunchKernel(fn, grid, dim3(kThreads), args, 0, stream) == hipSuccess ? BARQ_KV_OK
                                                                                 : BARQ_KV_ERR_LAUNCH;
}

template <int KIND>
const void* compress_fn_t(int ve) {
  if constexpr (KIND != BARQ_KV_FP32) {
    if (ve == 8) return (const void*)&compress_kernel<KIND, 8>;
  }
  switch (ve) {
    case 4: return (const void*)&compress_kernel<KIND, 4>;
    case 2: return (const void*)&compress_kernel<KIND, 2>;
    default: return (const void*)&compress_kernel<KIND, 1>;
  }
}

const void* compress_fn(int64_t kind, int ve) {
  return kind == BARQ_KV_BF16   ? compress_fn_t<BARQ_KV_BF16>(ve)
         : kind == BARQ_KV_FP16 ? compress_fn_t<BARQ_KV_FP16>(ve)
                                : compress_fn_t<BARQ_KV_FP32>(ve);
}

template <int KIND>
const void* compress_regs_fn_t(int nv) {
  switch (nv) {
    case 1: return (const void*)&compress_regs_kernel<KIND, 1>;
    case 2: return (const void*)&compress_regs_kernel<KIND, 2>;
    case 4: return (const void*)&compress_regs_kernel<KIND, 4>;
    default: return (const void*)&compress_regs_kernel<KIND, 8>;
  }
}

// The register-resident compress when the geometry admits it (2-byte elements in 16-byte
// vectors, G = kv_heads * head_dim / 8 dividing the workgroup, page_size * G / 256 vectors per
// thread in {1, 2, 4, 8} -- 16 would not stay in registers --, head_dim / 8 a power of two up
// to a wave), else null.
const void* compress_regs_fn(const barq_kv_pool* p, int64_t kind, int ve) {
  if (kind == BARQ_KV_FP32 || ve != 8) return nullptr;
  const int64_t C = p->kv_heads * p->head_dim, G = C / 8, vd = p->head_dim / 8;
  if (G < 1 || kThreads % G != 0 || vd > kWave || (vd & (vd - 1)) != 0 || (p->page_size * G) % kThreads != 0)
    return nullptr;
  const int64_t nv = p->page_size * G / kThreads;
  if (nv != 1 && nv != 2 && nv != 4 && nv != 8) return nullptr;
  return kind == BARQ_KV_BF16 ? compress_regs_fn_t<BARQ_KV_BF16>((int)nv)
                              : compress_regs_fn_t<BARQ_KV_FP16>((int)nv);
}

template <int KIND>
int launch_gather(int ve, int lpp, dim3 grid, GatherArgs* a, hipStream_t s) {
  const void* fn = (const void*)&gather_cold_kernel<KIND, 1>;
  if constexpr (KIND != BARQ_KV_FP32) {  // 8 two-byte elements: a 16-byte vector
    if (ve == 8) fn = (const void*)&gather_cold_kernel<KIND, 8>;
    if (ve == 8 && lpp == 1) fn = (const void*)&gather_cold_lanes_kernel<KIND, 1>;
    if (ve == 8 && lpp == 2) fn = (const void*)&gather_cold_lanes_kernel<KIND, 2>;
    if (ve == 8 && lpp == 4) fn = (const void*)&gather_cold_lanes_kernel<KIND, 4>;
  }
  if (ve == 4) fn = (const void*)&gather_cold_kernel<KIND, 4>;
  if (ve == 2) fn = (const void*)&gather_cold_kernel<KIND, 2>;
  void* args[] = {a};
  return hipLaunchKernel(fn, grid, dim3(kGatherThreads), args, 0, s) == hipSuccess ? BARQ_KV_OK : BARQ_KV_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int barq_kv_cold_reset(const barq_kv_pool* pool, const barq_kv_cold* cold, void* stream) {
  if (!cold_ok(pool, cold)) return BARQ_KV_ERR_INVALID;
  const int64_t blocks = (cold->num_cold + kThreads - 1) / kThreads;
  hipLaunchKernelGGL(cold_reset_kernel, dim3((uint32_t)blocks), dim3(kThreads), 0, (hipStream_t)stream,
                     cold_ptrs(cold), pool->ctrl);
  return hipGetLastError() == hipSuccess ? BARQ_KV_OK : BARQ_KV_ERR_LAUNCH;
}

}  // extern "C"

namespace {

// barq_kv_compress for the lengths the rows [0, batch) will have after `ahead` more tokens.
int compress_launch(const barq_kv_pool* pool, const barq_kv_cold* cold, int64_t batch, int64_t ahead,
                    void* stream) {
  if (!cold_ok(pool, cold) || batch < 0 || batch > pool->max_batch) return BARQ_KV_ERR_INVALID;
  if (batch == 0) return BARQ_KV_OK;
  CompressArgs a;
  a.p = *pool;
  a.c = cold_ptrs(cold);
  a.batch = (int32_t)batch;
  a.ahead = (int32_t)ahead;
  a.div_page = FastDiv::make((uint32_t)pool->page_size);
  a.div_dim = FastDiv::make((uint32_t)pool->head_dim);
  // widest vector along head_dim that every page row, code row and scale row admits
  const int64_t eb = pool->elem_bytes, D = pool->head_dim;
  const uint64_t bits = (uint64_t)(uintptr_t)pool->key_pages | (uint64_t)(uintptr_t)pool->value_pages;
  const uint64_t cbits = (uint64_t)(uintptr_t)cold->key_codes | (uint64_t)(uintptr_t)cold->value_codes |
                         (uint64_t)(uintptr_t)cold->key_scales;
  int ve = eb == 2 ? 8 : 4;
  while (ve > 1 && (D % ve || (bits & (uint64_t)(ve * eb - 1)) || (cbits & (uint64_t)(ve - 1)))) ve >>= 1;
  a.div_groups = FastDiv::make((uint32_t)(pool->kv_heads * D / ve));
  const void* fn = compress_regs_fn(pool, cold->element_type, ve);
  return launch(fn ? fn : compress_fn(cold->element_type, ve), dim3((uint32_t)batch), &a, (hipStream_t)stream);
}

// The update in two launches -- compress for the lengths the rows reach, then
// update_cold_lanes_kernel -- when it applies: tokens in [1, window], batch <= 64, two-byte
// elements whose token rows are 64, 128 or 256 vectors of 16 bytes, every address and stride
// 16-byte aligned (codes and key scales 8-byte), the output reaching the new tokens.  Returns -1
// (nothing launched) when it does not.
// Workgroups of a kGatherThreads-thread kernel resident at once on the current device (cached per
// slot and device; 0 when the runtime does not say).  Host threads may race on the cache, which
// only ever stores the one value a device gives.
int resident_tiles(const void* fn, int slot) {
  constexpr int kMaxDevices = 64;
  constexpr int kSlots = 6;
  static std::atomic<int> cached[kSlots][kMaxDevices];  // 0 = not queried yet
  int dev = 0;
  if (slot < 0 || slot >= kSlots || hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int v = cached[slot][dev].load(std::memory_order_relaxed);
  if (v == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kGatherThreads, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || per_cu <= 0 ||
        cus <= 0)
      return 0;
    v = per_cu * cus;
    cached[slot][dev].store(v, std::memory_order_relaxed);
  }
  return v;
}

int update_cold_fused(const barq_kv_pool* pool, const barq_kv_cold* cold, const void* ks, const void* vs,
                      int64_t batch, int64_t tokens, int64_t sb, int64_t sh, int64_t st, void* ko, void* vo,
                      int64_t seq_out, int64_t osb, int64_t osh, int64_t oss, int64_t flags, void* stream) {
  if (!cold_ok(pool, cold) || pool->elem_bytes != 2 || cold->element_type == BARQ_KV_FP32) return -1;
  if (batch < 1 || batch > kWave || batch > pool->max_batch || tokens < 1 || tokens > cold->window) return -1;
  const int64_t P = pool->page_size, H = pool->kv_heads, D = pool->head_dim;
  const int64_t cap = pool->max_blocks * P;
  if (seq_out < tokens || seq_out > cap) return -1;
  if (!ks || !vs || !ko || !vo || sb < 0 || sh < 0 || st < 0 || osb < 0 || osh < 0 || oss < 0) return -1;
  const uint64_t bits = (uint64_t)(uintptr_t)ko | (uint64_t)(uintptr_t)vo | (uint64_t)(osb * 2) |
                        (uint64_t)(osh * 2) | (uint64_t)(oss * 2) | (uint64_t)(D * 2) |
                        (uint64_t)(uintptr_t)pool->key_pages | (uint64_t)(uintptr_t)pool->value_pages |
                        (uint64_t)(uintptr_t)ks | (uint64_t)(uintptr_t)vs | (uint64_t)(sb * 2) |
                        (uint64_t)(sh * 2) | (uint64_t)(st * 2);
  const uint64_t code_bits = (uint64_t)(uintptr_t)cold->key_codes | (uint64_t)(uintptr_t)cold->value_codes |
                             (uint64_t)(uintptr_t)cold->key_scales | (uint64_t)D;
  if ((bits & 15) || (code_bits & 7)) return -1;
  const int64_t hd8 = H * D / 8;
  if (D % 8 != 0 || hd8 % kWave != 0 || (hd8 / kWave != 1 && hd8 / kWave != 2 && hd8 / kWave != 4) ||
      P * H * D > kI32Max)
    return -1;
  const int lpp = (int)(hd8 / kWave);
  if (!(flags & BARQ_KV_NO_COMPRESS)) {
    const int rc = compress_launch(pool, cold, batch, tokens, stream);
    if (rc != BARQ_KV_OK) return rc;
  }
  UpdateArgs u;
  GatherArgs& a = u.g;
  a.p = *pool;
  a.c = cold_ptrs(cold);
  a.out[0] = (char*)ko;
  a.out[1] = (char*)vo;
  a.osb = osb;
  a.osh = osh;
  a.oss = oss;
  a.batch = (int32_t)batch;
  a.seq_out = (int32_t)seq_out;
  a.nblk = (int32_t)((seq_out + P - 1) / P);
  a.from_device = (flags & BARQ_KV_SEQ_FROM_DEVICE) ? 1 : 0;
  a.div_head = FastDiv::make((uint32_t)(P * (D / 8)));
  a.div_dv = FastDiv::make((uint32_t)(D / 8));
  a.div_nblk = FastDiv::make((uint32_t)a.nblk);
  u.in[0] = (const char*)ks;
  u.in[1] = (const char*)vs;
  u.isb = sb;
  u.ish = sh;
  u.ist = st;
  u.tokens = (int32_t)tokens;
  const int64_t tiles = batch * a.nblk * 2;
  u.nsub = (int32_t)std::min<int64_t>(tiles, BARQ_KV_CTRL_SUBCOUNTERS);
  u.div_page = FastDiv::make((uint32_t)P);
  const bool f16 = cold->element_type == BARQ_KV_FP16;
  const void* fn = lpp == 1   ? (f16 ? (const void*)&update_cold_lanes_kernel<BARQ_KV_FP16, 1>
                                     : (const void*)&update_cold_lanes_kernel<BARQ_KV_BF16, 1>)
                   : lpp == 2 ? (f16 ? (const void*)&update_cold_lanes_kernel<BARQ_KV_FP16, 2>
                                     : (const void*)&update_cold_lanes_kernel<BARQ_KV_BF16, 2>)
                              : (f16 ? (const void*)&update_cold_lanes_kernel<BARQ_KV_FP16, 4>
                                     : (const void*)&update_cold_lanes_kernel<BARQ_KV_BF16, 4>);
  const int64_t resident = resident_tiles(fn, (lpp == 1 ? 0 : lpp == 2 ? 1 : 2) * 2 + (f16 ? 1 : 0));
  u.spaced = resident > 0 && tiles <= resident ? 1 : 0;
  void* args[] = {&u};
  return hipLaunchKernel(fn, dim3((uint32_t)tiles), dim3(kGatherThreads), args, 0, (hipStream_t)stream) == hipSuccess
             ? BARQ_KV_OK
             : BARQ_KV_ERR_LAUNCH;
}

}  // namespace

extern "C" {

int barq_kv_compress(const barq_kv_pool* pool, const barq_kv_cold* cold, int64_t batch, void* stream) {
  return compress_launch(pool, cold, batch, 0, stream);
}

int barq_kv_gather_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, void* key_out,
                        void* value_out, int64_t batch, int64_t seq_out, int64_t osb, int64_t osh,
                        int64_t oss, int64_t flags, void* stream) {
  if (!cold_ok(pool, cold) || batch < 0 || batch > pool->max_batch) return BARQ_KV_ERR_INVALID;
  if (flags & ~(int64_t)BARQ_KV_SEQ_FROM_DEVICE) return BARQ_KV_ERR_INVALID;
  const int64_t cap = pool->max_blocks * pool->page_size;
  if (seq_out < 0 || seq_out > cap) return BARQ_KV_ERR_INVALID;
  if (batch == 0 || seq_out == 0) return BARQ_KV_OK;
  if (!key_out || !value_out || osb < 0 || osh < 0 || oss < 0) return BARQ_KV_ERR_INVALID;
  const int64_t eb = pool->elem_bytes, D = pool->head_dim;
  // widest vector of VE elements every address and stride admits
  const uint64_t bits = (uint64_t)(uintptr_t)key_out | (uint64_t)(uintptr_t)value_out | (uint64_t)(osb * eb) |
                        (uint64_t)(osh * eb) | (uint64_t)(oss * eb) | (uint64_t)(D * eb) |
                        (uint64_t)(uintptr_t)pool->key_pages | (uint64_t)(uintptr_t)pool->value_pages;
  const uint64_t code_bits = (uint64_t)(uintptr_t)cold->key_codes | (uint64_t)(uintptr_t)cold->value_codes |
                             (uint64_t)(uintptr_t)cold->key_scales | (uint64_t)D;
  int ve = eb == 2 ? 8 : 4;
  while (ve > 1 && ((bits & (uint64_t)(ve * eb - 1)) || (code_bits & (uint64_t)(ve - 1)))) ve >>= 1;
  GatherArgs a;
  a.p = *pool;
  a.c = cold_ptrs(cold);
  a.out[0] = (char*)key_out;
  a.out[1] = (char*)value_out;
  a.osb = osb;
  a.osh = osh;
  a.oss = oss;
  a.batch = (int32_t)batch;
  a.seq_out = (int32_t)seq_out;
  a.nblk = (int32_t)((seq_out + pool->page_size - 1) / pool->page_size);
  a.from_device = (flags & BARQ_KV_SEQ_FROM_DEVICE) ? 1 : 0;
  a.div_head = FastDiv::make((uint32_t)(pool->page_size * (D / ve)));
  a.div_dv = FastDiv::make((uint32_t)(D / ve));
  a.div_nblk = FastDiv::make((uint32_t)a.nblk);
  const int64_t tiles = batch * a.nblk * 2;
  if (tiles > kI32Max) return BARQ_KV_ERR_INVALID;
  // Whole positions per wave: a token row of 64 * lpp vectors, and 32-bit offsets within a page
  const int64_t hd8 = pool->kv_heads * D / 8;
  const int lpp = (ve == 8 && D % 8 == 0 && hd8 % kWave == 0 &&
                   (hd8 / kWave == 1 || hd8 / kWave == 2 || hd8 / kWave == 4) &&
                   pool->page_size * pool->kv_heads * D <= kI32Max)
                      ? (int)(hd8 / kWave) : 0;
  hipStream_t s = (hipStream_t)stream;
  switch (cold->element_type) {
    case BARQ_KV_BF16: return launch_gather<BARQ_KV_BF16>(ve, lpp, dim3((uint32_t)tiles), &a, s);
    case BARQ_KV_FP16: return launch_gather<BARQ_KV_FP16>(ve, lpp, dim3((uint32_t)tiles), &a, s);
    default: return launch_gather<BARQ_KV_FP32>(ve, lpp, dim3((uint32_t)tiles), &a, s);
  }
}

int barq_kv_update_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, const void* key_states,
                        const void* value_states, int64_t batch, int64_t tokens, int64_t stride_b,
                        int64_t stride_h, int64_t stride_t, void* key_out, void* value_out,
                        int64_t seq_out, int64_t osb, int64_t osh, int64_t oss, int64_t flags,
                        void* stream) {
  if (!cold_ok(pool, cold)) return BARQ_KV_ERR_INVALID;
  if (flags & ~(int64_t)(BARQ_KV_SEQ_FROM_DEVICE | BARQ_KV_NO_COMPRESS)) return BARQ_KV_ERR_INVALID;
  const int fused = update_cold_fused(pool, cold, key_states, value_states, batch, tokens, stride_b, stride_h,
                                      stride_t, key_out, value_out, seq_out, osb, osh, oss, flags, stream);
  if (fused >= 0) return fused;
  int rc = barq_kv_append(pool, key_states, value_states, batch, tokens, stride_b, stride_h, stride_t, stream);
  if (rc == BARQ_KV_OK && !(flags & BARQ_KV_NO_COMPRESS)) rc = barq_kv_compress(pool, cold, batch, stream);
  if (rc == BARQ_KV_OK)
    rc = barq_kv_gather_cold(pool, cold, key_out, value_out, batch, seq_out, osb, osh, oss,
                             flags & BARQ_KV_SEQ_FROM_DEVICE, stream);
  return rc;
}

int barq_kv_crop_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, int64_t batch, int64_t max_length,
                      void* stream) {
  if (!cold_ok(pool, cold) || batch < 0 || batch > pool->max_batch) return BARQ_KV_ERR_INVALID;
  if (batch == 0) return BARQ_KV_OK;
  CropArgs a;
  a.p = *pool;
  a.c = cold_ptrs(cold);
  a.batch = (int32_t)batch;
  a.max_length = (int32_t)std::max<int64_t>(0, std::min<int64_t>(max_length, kI32Max));
  a.div_page = FastDiv::make((uint32_t)pool->page_size);
  const void* fn = cold->element_type == BARQ_KV_BF16   ? (const void*)&crop_cold_kernel<BARQ_KV_BF16>
                   : cold->element_type == BARQ_KV_FP16 ? (const void*)&crop_cold_kernel<BARQ_KV_FP16>
                                                        : (const void*)&crop_cold_kernel<BARQ_KV_FP32>;
  return launch(fn, dim3((uint32_t)batch), &a, (hipStream_t)stream);
}

int barq_kv_free_rows_cold(const barq_kv_pool* pool, const barq_kv_cold* cold, const int32_t* rows,
                           int64_t num_rows, void* stream) {
  if (!cold_ok(pool, cold) || num_rows < 0 || num_rows > pool->max_batch) return BARQ_KV_ERR_INVALID;
  if (num_rows == 0) return BARQ_KV_OK;
  if (!rows) return BARQ_KV_ERR_INVALID;
  FreeArgs a;
  a.p = *pool;
  a.c = cold_ptrs(cold);
  a.rows = rows;
  a.n = (int32_t)num_rows;
  a.div_page = FastDiv::make((uint32_t)pool->page_size);
  return launch((const void*)&free_rows_cold_kernel, dim3(1), &a, (hipStream_t)stream);
}

}  // extern "C"
