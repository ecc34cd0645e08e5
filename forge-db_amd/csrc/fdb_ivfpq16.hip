// IVF-PQ screening on the matrix cores with exact rescoring; the method and
// its bound are described in fdb_ivfpq16.hpp.
//
// pq16_decode_kernel   decoded residuals (codewords of each code, pq.rs:114-139
//                      inverted) to fp16 MFMA blocks, per list
// pq16_norms_kernel    |x^|^2 per code and the largest per list
// pq16_plan_kernel     each query's first lists and their buffer offsets
// pq16_count/offsets/scatter_kernel
//                      the probed (query, probe) pairs grouped by list
// pq16_dense_kernel    fp16 products of residuals and codes: every value of
//                      each query's first lists kept (stage A)
// pq16_thresh_kernel   the same products against each query's bound, the
//                      candidates appended (stage B)
// pq16_select_kernel   the bound d_k from the kept values
// pq16_classify_kernel the queries' flags and rescoring order
// pq16_rescore_kernel  exact table distances of the candidates in the
//                      reference's order (pq.rs:149-189 entries, :218-245 or
//                      :318-485 sums) and the top k, per query or per part
// pq16_merge_kernel    the parts' lists of a query merged
// pq16_stats_kernel    rescans and candidates, counted when read
#include "fdb_ivfpq16.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "fdb_device.hpp"

namespace fdb {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 8 halves as a native vector

constexpr int kT = 256;
// (query, probe) pairs per screening tile: 32 per wave, 4 waves
constexpr int kTilePairs = 128;
// Stage B: groups of 32 pairs per wave (tiles of 128 per group), and the
// waves per SIMD its registers are sized for.  Two groups where they fit
// three waves per SIMD (measured at 10M x 96, KC 6: 1.80 ms against 1.92
// with one group at four waves); at 1M x 128 (KC 8) two groups need the
// registers of two waves per SIMD and take 0.24 ms against 0.185 with one
// group at four.
constexpr int stage_b_groups(int KC) { return KC <= 6 ? 2 : 1; }
constexpr int stage_b_waves(int KC) { return KC <= 6 ? 3 : (KC <= 8 ? 4 : (KC <= 12 ? 3 : 2)); }
// Stage B's waves per workgroup and ring stages.  Measured at 1M x 128
// (KC 8): eight waves sharing a six- or eight-stage ring (tiles of 256
// pairs, two workgroups per CU) took 0.195 ms against 0.175-0.185 with four
// waves and three stages; four stages at four waves per SIMD, 0.183.
constexpr int stage_b_wgwaves(int KC) { return (void)KC, 4; }
constexpr int stage_b_stages(int KC) { return (void)KC, 3; }

uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }


// The wave's index in its workgroup as a wave-uniform value (scalar
// branches on it).
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

// Direct global-to-LDS loads: each lane's 16 (4) bytes from g land at
// lds + 16 (4) * lane; lds is wave-uniform.
__device__ __forceinline__ void lds_load16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* g, void* lds) { __builtin_amdgcn_global_load_lds(g, lds, 4, 0, 0); }
// s_waitcnt with an immediate; a workgroup barrier without a memory fence
// (the waits before it are explicit)
template <int IMM>
__device__ __forceinline__ void wait_imm() {
  __builtin_amdgcn_s_waitcnt(IMM);
}
__device__ __forceinline__ void bare_barrier() { __builtin_amdgcn_s_barrier(); }
// Scheduling hint: the N LDS reads of a block, then its N matrix products.
template <int N>
__device__ __forceinline__ void sched_reads_then_mfma() {
  __builtin_amdgcn_sched_group_barrier(0x100, N, 0);  // DS reads
  __builtin_amdgcn_sched_group_barrier(0x008, N, 0);  // MFMA
}


// WaveTopK registers for k: ceil(k / 64) rounded up to a power of two
int list_regs(int k) {
  int r = (k + 63) / 64, p = 1;
  while (p < r) p <<= 1;
  return p;
}

__global__ void pq16_fill_u32(uint32_t* __restrict__ p, uint64_t n, uint32_t v) {
  for (uint64_t i = (uint64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kT) p[i] = v;
}

// stats[0]: bits of the largest |codebook component| (non-finite values
// compare above every finite one).  Grid-stride, one atomic per wave.
__global__ __launch_bounds__(kT) void pq16_cb_stats_kernel(const float* __restrict__ cb, uint64_t n,
                                                           uint32_t* __restrict__ stats) {
  uint32_t m = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kT)
    m = max(m, __float_as_uint(cb[i]) & 0x7FFFFFFFu);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
  if ((threadIdx.x & 63) == 0) atomicMax(&stats[0], m);
}

// The list owning block B: the largest p < nlist with bo[p] <= B (lists
// without blocks share their successor's offset).
__device__ __forceinline__ uint32_t owner(const uint32_t* __restrict__ off, uint32_t nlist, uint32_t B) {
  uint32_t lo = 0, hi = nlist;  // off[lo] <= B < off[hi]
  while (hi - lo > 1) {
    const uint32_t mid = (lo + hi) >> 1;
    if (off[mid] <= B) lo = mid;
    else hi = mid;
  }
  return lo;
}

// Codewords padded to ds4 = dsub rounded up to 4 floats (zeros after).
__global__ __launch_bounds__(kT) void pq16_pad_cb_kernel(const float* __restrict__ cb, uint64_t nword, int dsub,
                                                         int ds4, float* __restrict__ out) {
  const uint64_t e = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (e >= nword * ds4) return;
  const uint64_t w = e / ds4;
  const int i = (int)(e - w * ds4);
  out[e] = i < dsub ? cb[w * dsub + i] : 0.0f;
}

// One workgroup (64*KC threads) per block; thread (kc, lane) writes the 8
// halves of its lane for k-chunk kc.
__global__ void pq16_decode_kernel(const float* __restrict__ cb, const uint8_t* __restrict__ codes,
                                   const uint32_t* __restrict__ list_off, const uint32_t* __restrict__ bo,
                                   uint32_t nlist, int M, int dsub, int KC, float scale,
                                   uint4* __restrict__ out) {
  const uint32_t B = blockIdx.x;
  const uint32_t p = owner(bo, nlist, B);
  const int kc = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t row = (B - bo[p]) * 32 + (lane & 31);
  const uint32_t len = list_off[p + 1] - list_off[p];
  const bool valid = row < len;
  const uint64_t i = (uint64_t)list_off[p] + row;
  const int D = M * dsub;
  _Float16 h[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int d = kc * 16 + 8 * (lane >> 5) + t;
    float v = 0.0f;
    if (valid && d < D) {
      const int m = d / dsub;
      const int e = d - m * dsub;
      v = cb[((uint64_t)m * 256 + codes[i * M + m]) * dsub + e] * scale;
    }
    h[t] = (_Float16)v;
  }
  uint4 w;
  w.x = (uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16);
  w.y = (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16);
  w.z = (uint32_t)__builtin_bit_cast(uint16_t, h[4]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[5]) << 16);
  w.w = (uint32_t)__builtin_bit_cast(uint16_t, h[6]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[7]) << 16);
  out[((uint64_t)B * KC + kc) * 64 + lane] = w;
}

// Thread per padded code slot: |x^|^2 in fp32 (FMA chain in dimension
// order; any order is within the bound's gamma_D) and the list maximum.
__global__ __launch_bounds__(kT) void pq16_norms_kernel(const float* __restrict__ cb,
                                                        const uint8_t* __restrict__ codes,
                                                        const uint32_t* __restrict__ list_off,
                                                        const uint32_t* __restrict__ bo, uint32_t nlist,
                                                        uint64_t nslots, int M, int dsub,
                                                        float* __restrict__ xnb, uint32_t* __restrict__ xmax2) {
  const uint64_t slot = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (slot >= nslots) return;
  const uint32_t B = (uint32_t)(slot >> 5);
  const uint32_t p = owner(bo, nlist, B);
  const uint32_t row = (B - bo[p]) * 32 + (uint32_t)(slot & 31);
  const uint32_t len = list_off[p + 1] - list_off[p];
  float s = 0.0f;
  if (row < len) {
    const uint64_t i = (uint64_t)list_off[p] + row;
    for (int m = 0; m < M; ++m) {
      const float* __restrict__ c = cb + ((uint64_t)m * 256 + codes[i * M + m]) * dsub;
      for (int e = 0; e < dsub; ++e) s = __builtin_fmaf(c[e], c[e], s);
    }
    atomicMax(&xmax2[p], __float_as_uint(s));
  }
  // slots past the list's end hold +inf: their screened value
  // fma(c, 0, +inf) never passes a finite threshold
  xnb[slot] = row < len ? s : f_inf();
}

// Blocks of full rows (Pq16Lists::build_rows): one workgroup (64*KC threads)
// per block, thread (kc, lane) writes the 8 halves of its lane for k-chunk kc.
__global__ void pq16_rows_kernel(const float* __restrict__ rows, const uint32_t* __restrict__ list_off,
                                 const uint32_t* __restrict__ bo, uint32_t nlist, int D, int KC, float scale,
                                 uint4* __restrict__ out) {
  const uint32_t B = blockIdx.x;
  const uint32_t p = owner(bo, nlist, B);
  const int kc = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t row = (B - bo[p]) * 32 + (lane & 31);
  const bool valid = row < list_off[p + 1] - list_off[p];
  const float* __restrict__ x = rows + ((uint64_t)list_off[p] + row) * D;
  _Float16 h[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int d = kc * 16 + 8 * (lane >> 5) + t;
    h[t] = (_Float16)(valid && d < D ? x[d] * scale : 0.0f);
  }
  uint4 w;
  w.x = (uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16);
  w.y = (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16);
  w.z = (uint32_t)__builtin_bit_cast(uint16_t, h[4]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[5]) << 16);
  w.w = (uint32_t)__builtin_bit_cast(uint16_t, h[6]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[7]) << 16);
  out[((uint64_t)B * KC + kc) * 64 + lane] = w;
}

// Thread per padded row slot: |x|^2 in fp32 (any order is within the bound's
// gamma_D), the list maximum, +inf past the list's end.
__global__ __launch_bounds__(kT) void pq16_row_norms_kernel(const float* __restrict__ rows,
                                                            const uint32_t* __restrict__ list_off,
                                                            const uint32_t* __restrict__ bo, uint32_t nlist,
                                                            uint64_t nslots, int D, float* __restrict__ xnb,
                                                            uint32_t* __restrict__ xmax2) {
  const uint64_t slot = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (slot >= nslots) return;
  const uint32_t B = (uint32_t)(slot >> 5);
  const uint32_t p = owner(bo, nlist, B);
  const uint32_t row = (B - bo[p]) * 32 + (uint32_t)(slot & 31);
  const bool valid = row < list_off[p + 1] - list_off[p];
  float s = 0.0f;
  if (valid) {
    const float* __restrict__ x = rows + ((uint64_t)list_off[p] + row) * D;
    for (int d = 0; d < D; ++d) s = __builtin_fmaf(x[d], x[d], s);
    atomicMax(&xmax2[p], __float_as_uint(s));
  }
  xnb[slot] = valid ? s : f_inf();
}

// ---- (query, probe) pairs by list ------------------------------------------
//
// A counting sort: workgroup w takes pairs [w*chunk, (w+1)*chunk) of the
// [nq][np] probe array.  pq16_count_kernel counts them per list in LDS and
// adds every nonzero count to cnt[list]; pq16_offsets_kernel turns cnt into
// each list's range of pairs (qoff) and of tiles; pq16_scatter_kernel
// recounts in LDS, claims the workgroup's range within each list by
// subtracting its count from cnt[list] (the value left is the range's
// start, and the subtractions leave cnt zero for the next search), and
// places every pair at qoff + range start + its LDS slot; it also writes
// the list of every tile (tl), for a share of the lists.  The order of a
// list's pairs follows the order of the atomics; the screening's results do
// not depend on it.  A pair (q, j) takes part when its list is valid and
// j < jlim[q] (jlim null: every probe).

constexpr uint32_t kHistMax = 8192;  // lists counted in LDS (32 KiB)
constexpr int kSortT = 1024;         // threads of a sorting workgroup
constexpr int kSortB = 8;            // pairs a sorting thread loads at once
constexpr int kSortWG = 256;         // sorting workgroups per stage (at most)
constexpr uint32_t kCB = 64;         // blocks of 32 codes per screening tile
constexpr uint32_t kCBDyn = 256;     // the same for size-sorted tiles taken from counters
constexpr uint32_t kCBMax = 256;     // at most (8 bits of a candidate entry)
constexpr uint32_t kXcd = 8;         // L2 domains (XCDs); workgroup b runs on XCD b % 8
constexpr uint32_t kXcdRun = 4;      // consecutive tiles given to one XCD (static tiles)
constexpr uint32_t kXcdRunDyn = 16;  // the same for dynamically taken tiles
constexpr int kNS = 4;               // one-block stages in stage A's LDS ring
constexpr uint32_t kLight = 256;     // candidate entries rescored by one wave (more: in parts)
constexpr uint32_t kPart = 256;      // entries of one part of a heavy query (a workgroup)
constexpr uint32_t kRound = 64;      // entries of one rescoring round

struct PairSet {
  const int32_t* probes;
  uint64_t nq;
  int np;
  const uint32_t* jlim;
  uint32_t nlist;
  uint64_t chunk;  // pairs per sorting workgroup
};

// The lists of pairs e + i*kSortT (i < kSortB) of a workgroup's range
// [., e1), ~0 for pairs past e1 or not taking part.  Every load is issued
// before the first is used (indices clamped into the range, e < e1).
// (pairs of a slice number below 2^32)
__device__ __forceinline__ void pair_lists(const PairSet& s, uint32_t e, uint32_t e1, uint32_t (&p)[kSortB]) {
  const uint32_t np = (uint32_t)s.np;
  int32_t v[kSortB];
  uint32_t lim[kSortB];
#pragma unroll
  for (int i = 0; i < kSortB; ++i) {
    const uint32_t ei = min(e + (uint32_t)(i * kSortT), e1 - 1);
    v[i] = s.probes[ei];
    lim[i] = s.jlim ? s.jlim[ei / np] : np;
  }
#pragma unroll
  for (int i = 0; i < kSortB; ++i) {
    const uint32_t ei = e + (uint32_t)(i * kSortT);
    const uint32_t j = ei - ei / np * np;
    p[i] = ei < e1 && j < lim[i] && v[i] >= 0 && (uint32_t)v[i] < s.nlist ? (uint32_t)v[i] : ~0u;
  }
}

// Both stages in one launch each (grid y = stage): 0 pairs the first lists
// (jlim), 1 every probe.  Stage st uses cnt + st*nlist, qoff and toff +
// st*(nlist+1), qlist + st*npr and desc + st*tl1.
struct PairStages {
  PairSet s0, s1;
  uint32_t blim0, blim1;  // blocks screened per list
  uint32_t tq0, tq1;      // pairs per tile
  uint32_t cb0, cb1;      // blocks per tile (at most kCBMax)
  uint32_t* cnt;          // [2][nlist], zero between searches
  uint32_t* qoff;
  uint32_t* toff;
  uint32_t* tcnt;         // [2][nlist] tiles of each list
  uint32_t* tctr;         // [2][kXcd] tile counters, zeroed by the offsets kernel
  uint2* qlist;
  uint4* desc;  // [tiles] tile descriptors (tile_work)
  uint64_t npr, tl1;
  uint32_t sort;  // tiles in descending order of size (else in list order)
};

__device__ __forceinline__ PairSet stage_set(const PairStages& ps, uint32_t st) { return st ? ps.s1 : ps.s0; }

// The workgroup's pairs [e0, e1) of its stage.
__device__ __forceinline__ void sort_range(const PairSet& s, uint32_t& e0, uint32_t& e1) {
  const uint64_t n = s.nq * (uint64_t)s.np;
  e0 = (uint32_t)min(n, blockIdx.x * s.chunk);
  e1 = (uint32_t)min(n, (blockIdx.x + 1) * s.chunk);
}

__global__ __launch_bounds__(kSortT) void pq16_count_kernel(PairStages ps) {
  __shared__ uint32_t hist[kHistMax];
  const PairSet s = stage_set(ps, blockIdx.y);
  uint32_t* __restrict__ cnt = ps.cnt + (uint64_t)blockIdx.y * s.nlist;
  for (uint32_t i = threadIdx.x; i < s.nlist; i += kSortT) hist[i] = 0;
  __syncthreads();
  uint32_t e0, e1;
  sort_range(s, e0, e1);
  for (uint32_t e = e0 + threadIdx.x; e < e1; e += kSortT * kSortB) {
    uint32_t p[kSortB];
    pair_lists(s, e, e1, p);
#pragma unroll
    for (int i = 0; i < kSortB; ++i)
      if (p[i] != ~0u) atomicAdd(&hist[p[i]], 1u);
  }
  __syncthreads();
  for (uint32_t i = threadIdx.x; i < s.nlist; i += kSortT) {
    const uint32_t h = hist[i];
    if (h) atomicAdd(&cnt[i], h);
  }
}

// Exclusive prefix of v over the workgroup's threads in thread order, added
// to carry (the running total, updated for the next call).  All threads call
// this; ws holds kSortT / 64 words.
__device__ __forceinline__ uint32_t block_prefix(uint32_t v, uint32_t* ws, uint32_t& carry) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t sc = v;  // inclusive wave scan
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t u = (uint32_t)__shfl_up((int)sc, off);
    if (lane >= off) sc += u;
  }
  if (lane == 63) ws[wave] = sc;
  __syncthreads();
  uint32_t pre = carry, tot = carry;
  for (int w = 0; w < kSortT / 64; ++w) {
    pre += w < wave ? ws[w] : 0u;
    tot += ws[w];
  }
  __syncthreads();
  carry = tot;
  return pre + sc - v;
}

// One workgroup of kSortT threads per stage, thread t taking lists t +
// u*kSortT.
//   qoff = exclusive prefix of cnt in list order (qoff[nlist] the total).
//   tiles_p = ceil(cnt_p / tq) * ceil(min(nb_p, blim) / cb) (nb_p = bo[p+1] -
//   bo[p]); with sort, the tile ranges are laid out in descending order of
//   the list's full tile (min(nb_p, blim, cb) blocks x min(groups_p, tq/32)
//   groups of 32 pairs), so that workgroups taking tiles in order meet the
//   longest first and the shortest last (the order within equal sizes
//   follows the LDS atomics); else in list order.  toff[p] = the list's first
//   tile, tcnt[p] = its tiles, toff[nlist] = the total.  The stage's tile
//   counters are zeroed.
__global__ __launch_bounds__(kSortT) void pq16_offsets_kernel(PairStages ps, const uint32_t* __restrict__ bo) {
  constexpr int kU = kHistMax / kSortT;
  constexpr uint32_t kKeys = kCBMax * 8 + 1;  // tile sizes 0 .. 256 blocks x 8 groups
  const uint32_t stage = blockIdx.x;
  const uint32_t nlist = ps.s0.nlist;
  const uint32_t blim = stage ? ps.blim1 : ps.blim0;
  const uint32_t tq = stage ? ps.tq1 : ps.tq0;
  const uint32_t cb = stage ? ps.cb1 : ps.cb0;
  const bool sort = ps.sort != 0;
  const uint32_t* __restrict__ cnt = ps.cnt + (uint64_t)stage * nlist;
  uint32_t* __restrict__ qoff = ps.qoff + (uint64_t)stage * (nlist + 1);
  uint32_t* __restrict__ toff = ps.toff + (uint64_t)stage * (nlist + 1);
  uint32_t* __restrict__ tcnt = ps.tcnt + (uint64_t)stage * nlist;
  __shared__ uint32_t ws[kSortT / 64];
  __shared__ uint32_t hist[kKeys];
  __shared__ uint32_t tbr[kHistMax];  // tiles by rank, then their prefix
  const int tid = threadIdx.x;
  if (tid < (int)kXcd) ps.tctr[stage * kXcd + tid] = 0u;
  // (the histogram ranks the lists by tile size; unsorted, a list's rank is
  // its index and the histogram is skipped)
  if (sort)
    for (uint32_t i = tid; i < kKeys; i += kSortT) hist[i] = 0;
  // every list's count and block count first
  uint32_t c[kU], nb[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const uint32_t i = min((uint32_t)(u * kSortT + tid), nlist - 1);
    c[u] = cnt[i];
    nb[u] = bo[i + 1] - bo[i];
  }
  __syncthreads();
  // pair offsets in list order; tile counts and size keys, ranked by key
  uint32_t carry = 0, t[kU], key[kU], rin[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const uint32_t i = u * kSortT + tid;
    const uint32_t cu = i < nlist ? c[u] : 0u;
    const uint32_t nbl = min(nb[u], blim);
    t[u] = (cu + tq - 1) / tq * ((nbl + cb - 1) / cb);
    key[u] = t[u] ? min(nbl, cb) * min((cu + 31) / 32, tq / 32) : 0u;
    if ((uint32_t)(u * kSortT) < nlist) {  // workgroup-uniform
      const uint32_t pre = block_prefix(cu, ws, carry);
      if (i < nlist) qoff[i] = pre;
    }
    rin[u] = sort && i < nlist ? atomicAdd(&hist[key[u]], 1u) : 0u;
  }
  if (tid == 0) qoff[nlist] = carry;
  __syncthreads();
  // bucket starts in descending key order (wave 0: lane l sums keys
  // kKeys-1-9l .. kKeys-9-9l)
  if (sort && tid < 64) {
    constexpr int kPer = (kKeys + 63) / 64;
    uint32_t sum = 0;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int kk = (int)kKeys - 1 - (tid * kPer + e);
      sum += kk >= 0 ? hist[kk] : 0u;
    }
    uint32_t sc = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t u = (uint32_t)__shfl_up((int)sc, off);
      if (tid >= off) sc += u;
    }
    uint32_t run = sc - sum;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int kk = (int)kKeys - 1 - (tid * kPer + e);
      if (kk >= 0) {
        const uint32_t h = hist[kk];
        hist[kk] = run;
        run += h;
      }
    }
  }
  __syncthreads();
  uint32_t rank[kU];
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const uint32_t i = u * kSortT + tid;
    rank[u] = i >= nlist ? 0u : sort ? hist[key[u]] + rin[u] : i;
    if (i < nlist) tbr[rank[u]] = t[u];
  }
  __syncthreads();
  // tile offsets in rank order
  carry = 0;
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const uint32_t r = u * kSortT + tid;
    if ((uint32_t)(u * kSortT) < nlist) {  // workgroup-uniform
      const uint32_t v = r < nlist ? tbr[r] : 0u;
      const uint32_t pre = block_prefix(v, ws, carry);
      if (r < nlist) tbr[r] = pre;
    }
  }
  __syncthreads();
#pragma unroll
  for (int u = 0; u < kU; ++u) {
    const uint32_t i = u * kSortT + tid;
    if (i < nlist) {
      toff[i] = tbr[rank[u]];
      tcnt[i] = t[u];
    }
  }
  if (tid == 0) toff[nlist] = carry;
}

__global__ __launch_bounds__(kSortT) void pq16_scatter_kernel(PairStages ps, const uint32_t* __restrict__ bo) {
  __shared__ uint32_t hist[kHistMax];
  const PairSet s = stage_set(ps, blockIdx.y);
  uint32_t* __restrict__ cnt = ps.cnt + (uint64_t)blockIdx.y * s.nlist;
  const uint32_t* __restrict__ qoff = ps.qoff + (uint64_t)blockIdx.y * (s.nlist + 1);
  uint2* __restrict__ qlist = ps.qlist + blockIdx.y * ps.npr;
  const uint32_t np = (uint32_t)s.np;
  for (uint32_t i = threadIdx.x; i < s.nlist; i += kSortT) hist[i] = 0;
  // desc[t] = the descriptor of tile t, for the workgroup's share of the
  // lists: lane j of wave w takes list b + j*16 + w of each run b of 1024,
  // and all the wave's lanes write each one's tiles (the first run's tile
  // ranges loaded now, written at the end)
  const uint32_t* __restrict__ toff = ps.toff + (uint64_t)blockIdx.y * (s.nlist + 1);
  const uint32_t* __restrict__ tcnt = ps.tcnt + (uint64_t)blockIdx.y * s.nlist;
  const uint32_t per = (s.nlist + gridDim.x - 1) / gridDim.x;
  const uint32_t l0 = blockIdx.x * per, l1 = min(s.nlist, l0 + per);
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t r = lane * (kSortT / 64) + (threadIdx.x >> 6);
  uint32_t lo0 = 0, hi0 = 0;
  if (l0 + r < l1) {
    lo0 = toff[l0 + r];
    hi0 = lo0 + tcnt[l0 + r];
  }
  __syncthreads();
  uint32_t e0, e1;
  sort_range(s, e0, e1);
  // the counts (the first batch's lists kept)
  uint32_t p0[kSortB];
  const uint32_t f = e0 + threadIdx.x;
  if (f < e1) {
    pair_lists(s, f, e1, p0);
#pragma unroll
    for (int i = 0; i < kSortB; ++i)
      if (p0[i] != ~0u) atomicAdd(&hist[p0[i]], 1u);
  }
  for (uint32_t e = f + kSortT * kSortB; e < e1; e += kSortT * kSortB) {
    uint32_t p[kSortB];
    pair_lists(s, e, e1, p);
#pragma unroll
    for (int i = 0; i < kSortB; ++i)
      if (p[i] != ~0u) atomicAdd(&hist[p[i]], 1u);
  }
  __syncthreads();
  // the workgroup's range of each list: hist becomes its next position
  for (uint32_t i = threadIdx.x; i < s.nlist; i += kSortT) {
    const uint32_t h = hist[i];
    if (h) hist[i] = qoff[i] + atomicSub(&cnt[i], h) - h;
  }
  __syncthreads();
  if (f < e1) {
#pragma unroll
    for (int i = 0; i < kSortB; ++i)
      if (p0[i] != ~0u) {
        const uint32_t e = f + (uint32_t)(i * kSortT);
        const uint32_t q = e / np;
        qlist[atomicAdd(&hist[p0[i]], 1u)] = make_uint2(q, e - q * np);
      }
  }
  for (uint32_t e = f + kSortT * kSortB; e < e1; e += kSortT * kSortB) {
    uint32_t p[kSortB];
    pair_lists(s, e, e1, p);
#pragma unroll
    for (int i = 0; i < kSortB; ++i)
      if (p[i] != ~0u) {
        const uint32_t ei = e + (uint32_t)(i * kSortT);
        const uint32_t q = ei / np;
        qlist[atomicAdd(&hist[p[i]], 1u)] = make_uint2(q, ei - q * np);
      }
  }
  uint4* __restrict__ desc = ps.desc + blockIdx.y * ps.tl1;
  const uint32_t tq = blockIdx.y ? ps.tq1 : ps.tq0, cb = blockIdx.y ? ps.cb1 : ps.cb0;
  const uint32_t blim = blockIdx.y ? ps.blim1 : ps.blim0;
  for (uint32_t b = l0; b < l1; b += kSortT) {
    uint32_t lo = lo0, hi = hi0;
    if (b != l0) {
      lo = hi = 0;
      if (b + r < l1) {
        lo = toff[b + r];
        hi = lo + tcnt[b + r];
      }
    }
    for (uint64_t m = __ballot(hi != lo); m; m &= m - 1) {
      const int l = __builtin_ctzll(m);
      const uint32_t al = (uint32_t)__builtin_amdgcn_readlane((int)lo, l);
      const uint32_t nl = (uint32_t)__builtin_amdgcn_readlane((int)(hi - lo), l);
      const uint32_t li = (uint32_t)__builtin_amdgcn_readlane((int)(b + r), l);
      const uint32_t qb = qoff[li], qe = qoff[li + 1], b0 = bo[li];
      const uint32_t nb = min(bo[li + 1] - b0, blim);
      const uint32_t nqt = (qe - qb + tq - 1) / tq;
      for (uint32_t v = lane; v < nl; v += 64) {
        const uint32_t chunk = v / nqt, pt = v - chunk * nqt;
        desc[al + v] = make_uint4(li | (min(cb, nb - chunk * cb) << 16), qb + pt * tq, qe, b0 + chunk * cb);
      }
    }
  }
}

// Thread per query: the first probes whose lists hold at least k codes
// (jlim), each one's 32-aligned offset into the query's buffer of screened
// values (offA [nq][np]; nothing past capA is kept), the buffer entries
// written (nA, padding included) and the codes among them (nreal).
__global__ __launch_bounds__(kT) void pq16_plan_kernel(const int32_t* __restrict__ probes, uint64_t nq, int np,
                                                       uint32_t nlist, const uint32_t* __restrict__ list_off,
                                                       int k, uint32_t capA, uint32_t* __restrict__ jlim,
                                                       uint32_t* __restrict__ offA, uint32_t* __restrict__ nA,
                                                       uint32_t* __restrict__ nreal, uint32_t* __restrict__ ccnt,
                                                       int* __restrict__ force, float* __restrict__ epsA,
                                                       uint32_t* __restrict__ counters) {
  const uint64_t q0 = (uint64_t)blockIdx.x * kT;
  const uint64_t q = q0 + threadIdx.x;
  if (q < 4) counters[q] = 0;
  // the workgroup's bounds start clear (coalesced)
  const uint64_t e1 = min(nq, q0 + kT) * (uint64_t)np;
  for (uint64_t e = q0 * np + threadIdx.x; e < e1; e += kT) epsA[e] = 0.0f;
  if (q >= nq) return;
  ccnt[q] = 0;  // the query's counters start clear
  force[q] = 0;
  // the first kPre probes' list lengths loaded together
  constexpr int kPre = 4;
  uint32_t len[kPre];
  {
    int32_t p[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) p[j] = probes[q * np + min(j, np - 1)];
#pragma unroll
    for (int j = 0; j < kPre; ++j) {
      const bool ok = p[j] >= 0 && (uint32_t)p[j] < nlist;
      const uint32_t pc = ok ? (uint32_t)p[j] : 0u;
      const uint32_t a0 = list_off[pc], a1 = list_off[pc + 1];
      len[j] = ok ? a1 - a0 : 0u;  // an invalid probe: no codes
    }
  }
  uint64_t cum = 0, real = 0;
  uint32_t J = 0;
  for (int j = 0; j < np; ++j) {
    if (real >= (uint64_t)k || cum >= capA) break;
    uint64_t n;
    if (j < kPre) {
      n = len[0];
#pragma unroll
      for (int u = 1; u < kPre; ++u) n = j == u ? len[u] : n;
    } else {
      const int32_t p = probes[q * np + j];
      n = p >= 0 && (uint32_t)p < nlist ? list_off[p + 1] - list_off[p] : 0;
    }
    offA[q * np + j] = (uint32_t)cum;
    J = (uint32_t)j + 1;
    real += std::min<uint64_t>(n, capA - cum);
    cum += (n + 31) / 32 * 32;
  }
  jlim[q] = J;
  nA[q] = (uint32_t)std::min<uint64_t>(cum, capA);
  nreal[q] = (uint32_t)real;
}

// ---- screening --------------------------------------------------------------

struct ScreenArgs {
  const float* queries;
  int D;
  int vec;  // D = 16 * KC and 16-byte aligned query and centroid rows
  const float* centroids;
  const uint32_t* list_off;
  const uint32_t* bo;
  const uint4* data;
  const float* xnb;
  const uint32_t* xmax2;
  uint32_t nlist;
  int np;
  int xexp;
  const uint32_t* qoff;
  const uint32_t* toff;
  const uint4* desc;  // tile descriptors: list | blocks << 16, first pair, list's pair end, first block
  const uint2* qlist;
  uint32_t blim;  // blocks screened per list at most
  uint32_t cb;    // blocks per tile (at most kCBMax)
  uint32_t* tctr;  // the stage's kXcd tile counters (zero at launch)
  uint32_t dyn;    // tiles taken from the counters (else a static stride)
  uint32_t run;    // consecutive tiles per XCD
  // dense mode: every kept value to bufA[q][offA[q][j] + row] (< capA) and
  // the pair's bound to epsA[q][j]
  float* bufA;
  const uint32_t* offA;
  float* epsA;
  uint32_t capA;
  // threshold mode: codes with s <= dkA[q] + eps become candidates
  const float* dkA;
  uint32_t* ccnt;
  uint2* cand;
  uint32_t cap;
  int* force;
  float c_dot, c_sq, cabs;  // pq16_eps coefficients
};

// |s - d| <= c_dot*|r|*X' + c_sq*(|r| + X')^2 (+ a floor), X' = X + cabs; see
// pq16_eps_coeffs for the derivation.
__device__ __forceinline__ float pq16_eps(float rnorm, float X, const ScreenArgs& a) {
  const float Xp = X + a.cabs;
  const float t = rnorm + Xp;
  return a.c_dot * rnorm * Xp + a.c_sq * t * t + 1e-30f;
}

// a + b rounded up past the exact sum (a, b >= 0)
__device__ __forceinline__ float add_up(float a, float b) {
  const float t = a + b;
  return t + t * 0x1p-22f;
}

// Tiles: list p owns toff[p] .. toff[p+1]: ceil(pairs_p / 128) pair tiles
// (fastest) times ceil(min(blocks_p, blim) / cb) block chunks; workgroups
// of four waves stride over the tiles.  In a tile, wave w takes pairs
// [32w, 32w+32); with fewer than four groups of 32 pairs, each group has
// split waves, which take every split-th block of the chunk.  Tiles of one
// list chunk (its pair tiles are consecutive) read the same blocks: runs of
// kXcdRun consecutive tiles go to workgroups b, b + 8, b + 16, ... of one
// XCD, dispatched together, so the repeat reads hit that XCD's L2 (a
// bijection on each round of gridDim.x tiles, a multiple of kXcd * kXcdRun).
struct TileWork {
  uint32_t p, nblk, babs, q0, qend;
  int split, phase;
  bool busy;   // wave-uniform: the wave has pairs
  uint32_t q1;  // a second group of 32 pairs (tiles of 256 pairs)
  bool busy1;  // wave-uniform: the wave has the second group
};

// The c-th tile of the workgroup's XCD (x = blockIdx.x % kXcd): runs of
// `run` consecutive tiles per XCD (tiles of one list chunk are consecutive,
// so their repeat block reads can hit that XCD's L2).
__device__ __forceinline__ uint32_t xcd_tile(uint32_t c, uint32_t run) {
  return ((c / run) * kXcd + blockIdx.x % kXcd) * run + c % run;
}

// The workgroup's tile loop: body(t) for each tile it takes.  A workgroup's
// first tile is c = blockIdx.x / kXcd of its XCD.  Static (dyn 0): then
// every (gridDim.x / kXcd)-th of its XCD's tiles.  Dynamic (dyn 1, a grid of
// resident workgroups): the next ones come from the XCD's counter, so
// workgroups that finish early take more; thread 0 claims the next tile
// while the current one runs (the atomic is older than every load of the
// tile, so the ring's waits cover it) and one barrier per tile passes it on.
template <class Body>
__device__ __forceinline__ void for_tiles(uint32_t ntiles, uint32_t* __restrict__ tctr, uint32_t dyn, uint32_t run,
                                          uint32_t* s_next, Body&& body) {
  const uint32_t per = gridDim.x / kXcd;
  uint32_t c = blockIdx.x / kXcd;
  for (uint32_t t = xcd_tile(c, run); t < ntiles;) {
    uint32_t nxt = 0;
    if (dyn && threadIdx.x == 0) nxt = atomicAdd(&tctr[blockIdx.x % kXcd], 1u);
    body(t);
    if (dyn) {
      if (threadIdx.x == 0) *s_next = nxt;
      __syncthreads();
      c = per + *s_next;
    } else {
      c += per;
    }
    t = xcd_tile(c, run);
  }
}

// Tiles of TQ pairs for WV waves: wave w takes pairs [32w, 32w + 32) of the
// tile (and group w + WV when TQ / 32 > WV, with two groups per wave); with
// fewer groups than waves, each group has split waves, which take every
// split-th block of the chunk.  One descriptor load gives the tile.
template <uint32_t TQ, int WV>
__device__ __forceinline__ TileWork tile_work(const ScreenArgs& a, uint32_t t, int wave) {
  static_assert(TQ / 32 == WV || TQ / 32 == 2 * WV, "one or two groups of 32 pairs per wave");
  TileWork w;
  const uint4 d = a.desc[t];
  w.p = d.x & 0xFFFFu;
  w.nblk = d.x >> 16;
  w.babs = d.w;
  w.qend = d.z;
  const uint32_t tq0 = d.y;
  const uint32_t ngr = min((w.qend - tq0 + 31) / 32, TQ / 32);
  const uint32_t ng = min(ngr, (uint32_t)WV);
  const uint32_t gp = ng <= 1 ? 1u : ng <= 2 ? 2u : ng <= 4 ? 4u : 8u;  // groups rounded up to a power of 2
  w.split = WV / (int)min(gp, (uint32_t)WV);
  w.phase = wave % w.split;
  w.q0 = tq0 + (uint32_t)(wave / w.split) * 32;
  w.busy = w.q0 < w.qend;
  w.q1 = tq0 + (uint32_t)(wave + WV) * 32;
  w.busy1 = ngr > (uint32_t)WV && w.q1 < w.qend;  // split is 1 then
  return w;
}

// The B operand of the lane's (query, probe) pair: lane l holds the
// residual r = q - c_p of pair l%32 (the reference's residual, fp32) on
// dimensions 16kc + 8(l/32) .. +7, scaled by 2^er so that its largest
// component lies in [2^12, 2^13), as halves; rn = |r|^2 in fp32.  bad when
// the residual does not fit fp16 (non-finite norm, er beyond +-100).
template <int KC>
struct PairOperand {
  v8h bq[KC];
  float rn;
  int er;
  bool bad;
};

template <int KC>
__device__ __forceinline__ void pair_operand(const ScreenArgs& a, uint32_t q, uint32_t p, int half,
                                             PairOperand<KC>& o) {
  const float* __restrict__ qp = a.queries + (uint64_t)q * a.D;
  // full vectors (no centroids): the residual is the query itself
  const float* __restrict__ cp = a.centroids ? a.centroids + (uint64_t)p * a.D : qp;
  const float cs = a.centroids ? 1.0f : 0.0f;
  float r[KC][8];
  if (a.vec) {  // whole k-chunks, 16-byte aligned rows: 16-byte loads
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int h4 = 0; h4 < 2; ++h4) {
        const int d = kc * 16 + 8 * half + 4 * h4;
        const float4 x = *reinterpret_cast<const float4*>(qp + d);
        const float4 c = *reinterpret_cast<const float4*>(cp + d);
        r[kc][4 * h4] = x.x - cs * c.x;
        r[kc][4 * h4 + 1] = x.y - cs * c.y;
        r[kc][4 * h4 + 2] = x.z - cs * c.z;
        r[kc][4 * h4 + 3] = x.w - cs * c.w;
      }
  } else {
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int d = kc * 16 + 8 * half + i;
        r[kc][i] = d < a.D ? qp[d] - cs * cp[d] : 0.0f;
      }
  }
  float mx = 0.0f, rn = 0.0f;
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      mx = fmaxf(mx, __builtin_fabsf(r[kc][i]));
      rn = __builtin_fmaf(r[kc][i], r[kc][i], rn);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  rn = rn + __shfl_xor(rn, 32);
  int er = 0;
  if (mx > 0.0f) {
    int E;
    (void)frexpf(mx, &E);
    er = 13 - E;  // mx * 2^er in [2^12, 2^13)
  }
  const float sc = ldexpf(1.0f, er);
#pragma unroll
  for (int kc = 0; kc < KC; ++kc)
#pragma unroll
    for (int i = 0; i < 8; ++i) o.bq[kc][i] = (_Float16)(r[kc][i] * sc);
  o.rn = rn;
  o.er = er;
  o.bad = !(rn <= 3.0e38f) || er > 100 || er < -100;
}

// The 16 |x^|^2 values of a lane's rows in a block (rows 8(i/4) + 4(l/32) +
// i%4) from the block's 32 norms in LDS.
__device__ __forceinline__ void block_norms(const float* __restrict__ sx, int half, float* xs) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const float4 x4 = *reinterpret_cast<const float4*>(sx + 8 * g + 4 * half);
    xs[4 * g] = x4.x;
    xs[4 * g + 1] = x4.y;
    xs[4 * g + 2] = x4.z;
    xs[4 * g + 3] = x4.w;
  }
}

// The LDS ring of one workgroup: NS one-block stages, each the block's KC
// A-operand chunks and its 32 norms.
template <int KC, int NS, int WV>
struct Ring {
  v4u blk[NS][KC * 64];
  float xn[NS][64];
  v4u dummy[(KC + WV - 1) / WV * WV > KC ? 64 : 1];
  float dxn[64];
};

// Streams the nst blocks of a tile (A operands at A, norms at XN, both at
// the tile's first block) through the ring by direct global-to-LDS loads;
// block s lands in stage s % NS.  Every wave issues kUW + 1 loads per block
// (k-chunks w, w + WV, ...; wave 0 also the block's norms; spare loads
// re-read into a dummy buffer), so waiting for all but the newest NS - 2
// blocks' loads is one immediate count (loads issued after them only make
// it wait for more), and a workgroup barrier then frees the previous stage.
// Blocks past the end re-read the last block.  ring_begin issues the first
// NS - 1 blocks (before the pair operands are loaded, so that their latency
// overlaps); ring_run streams the rest: step(stage, norms, s) runs on the
// waves whose pairs take block s.  All waves call both.
template <int KC, int NS, int WV>
struct RingStream {
  static constexpr int kUW = (KC + WV - 1) / WV;
  Ring<KC, NS, WV>& ring;
  const char* __restrict__ Ab;
  const char* __restrict__ Xb;
  uint32_t nst;
  int wave;
  uint32_t lo16, lo4;
  __device__ __forceinline__ RingStream(Ring<KC, NS, WV>& r, const v4u* A, const float* XN, uint32_t n, int wv,
                                        int lane)
      : ring(r), Ab(reinterpret_cast<const char*>(A)), Xb(reinterpret_cast<const char*>(XN)), nst(n), wave(wv),
        lo16((uint32_t)lane * 16), lo4((uint32_t)(lane & 31) * 4) {}
  __device__ __forceinline__ void issue(int buf, uint32_t sblk) {
    const uint32_t bl = min(sblk, nst - 1);
#pragma unroll
    for (int i = 0; i < kUW; ++i) {
      const int u = wave + WV * i;
      if (u < KC)
        lds_load16(Ab + ((uint64_t)bl * KC + u) * 1024 + lo16, &ring.blk[buf][u * 64]);
      else
        lds_load16(Ab + (uint64_t)bl * KC * 1024 + lo16, &ring.dummy[0]);
    }
    if (wave == 0)
      lds_load4(Xb + (uint64_t)bl * 128 + lo4, &ring.xn[buf][0]);
    else
      lds_load4(Xb + (uint64_t)bl * 128 + lo4, &ring.dxn[0]);
  }
  __device__ __forceinline__ void begin() {
#pragma unroll
    for (int i = 0; i < NS - 1; ++i) issue(i, (uint32_t)i);
  }
  template <class Step>
  __device__ __forceinline__ void run(const TileWork& w, Step&& step) {
    // s_waitcnt immediates (vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt
    // at their maxima): all but the newest NS - 2 blocks' loads, and all
    constexpr int kRingLoads = (NS - 2) * (kUW + 1);
    constexpr int kWaitRing = (kRingLoads & 15) | ((kRingLoads >> 4) << 14) | 0x70 | 0xF00;
    constexpr int kWaitAll = 0x70 | 0xF00;
    for (uint32_t s = 0; s < nst;) {
#pragma unroll
      for (int buf = 0; buf < NS; ++buf) {
        if (s < nst) {
          wait_imm<kWaitRing>();  // this wave's loads of block s have landed
          bare_barrier();         // everyone's have; stage (s-1) % NS is free
          issue((buf + NS - 1) % NS, s + NS - 1);
          if (w.busy && (int)(s % w.split) == w.phase) step(ring.blk[buf], ring.xn[buf], s);
          ++s;
        }
      }
    }
    wait_imm<kWaitAll>();  // spare loads of the ring's tail
    bare_barrier();        // the ring is free for the next tile
  }
};

// Stage A: every screened value s = fma(-2^(1-er-xexp), acc, |r|^2 + |x^|^2)
// of the pair's first lists goes to the pair's 32-aligned range of the
// query's buffer (+inf past the list's end, nothing past capA), four rows
// per 16-byte store, and the pair's bound to epsA.  D[r] of a product is
// code 8(r/4) + 4(l/32) + r%4 of the block against pair l%32.
template <int KC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void pq16_dense_kernel(ScreenArgs a) {
  __shared__ Ring<KC, kNS, 4> ring;
  const int lane = threadIdx.x & 63;
  const int wave = wave_index();
  const int col = lane & 31;
  const int half = lane >> 5;
  __shared__ uint32_t s_next;
  const uint32_t ntiles = a.toff[a.nlist];
  for_tiles(ntiles, a.tctr, a.dyn, a.run, &s_next, [&](uint32_t t) {
    const TileWork w = tile_work<kTilePairs, 4>(a, t, wave);
    const uint32_t p = w.p;
    RingStream<KC, kNS, 4> rs(ring, reinterpret_cast<const v4u*>(a.data) + (uint64_t)w.babs * KC * 64,
                              a.xnb + (uint64_t)w.babs * 32, w.nblk, wave, lane);
    rs.begin();
    const bool qv = w.busy && w.q0 + (uint32_t)col < w.qend;
    // lanes past the tile's pairs repeat its last pair, so that every load
    // is in bounds without a branch per load (qv keeps them inactive)
    const uint2 e = a.qlist[min(w.q0 + (uint32_t)col, w.qend - 1)];
    const uint32_t q = e.x, j = e.y;
    PairOperand<KC> op;
    pair_operand<KC>(a, q, p, half, op);
    const bool act = qv && !op.bad;
    if (qv && op.bad && half == 0) atomicOr(&a.force[q], 1);
    uint32_t o = 0;  // buffer offset of the pair
    if (act) {
      const float rnorm = sqrtf(op.rn) * (1.0f + 0x1p-16f);
      const float X = sqrtf(__uint_as_float(a.xmax2[p])) * (1.0f + 0x1p-16f);
      o = a.offA[(uint64_t)q * a.np + j];
      if (half == 0 && w.babs == a.bo[p]) a.epsA[(uint64_t)q * a.np + j] = pq16_eps(rnorm, X, a);
    }
    const float cneg = -ldexpf(1.0f, 1 - op.er - a.xexp);
    const float rn = op.rn;
    const uint32_t bb = w.babs - a.bo[p];  // the tile's first block in the list
    const uint32_t len = a.list_off[p + 1] - a.list_off[p];
    rs.run(w, [&](const v4u* __restrict__ sa, const float* __restrict__ sx, uint32_t sb) {
      const uint32_t b = bb + sb;
      // every k-chunk read from LDS before the first product: one LDS
      // round trip per block instead of one per pair of products
      v4u av[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) av[kc] = sa[kc * 64 + lane];
      v16f acc = {};
#pragma unroll
      for (int kc = 0; kc < KC; ++kc)
        acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, av[kc]), op.bq[kc], acc, 0, 0, 0);
      sched_reads_then_mfma<KC>();
      float xs[16];
      block_norms(sx, half, xs);
      if (act) {
        const uint32_t rowb = b * 32 + 4 * half;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t row = rowb + 8 * g;
          if (o + row < a.capA) {
            float4 v;
            v.x = row + 0 < len ? __builtin_fmaf(cneg, acc[4 * g + 0], rn + xs[4 * g + 0]) : f_inf();
            v.y = row + 1 < len ? __builtin_fmaf(cneg, acc[4 * g + 1], rn + xs[4 * g + 1]) : f_inf();
            v.z = row + 2 < len ? __builtin_fmaf(cneg, acc[4 * g + 2], rn + xs[4 * g + 2]) : f_inf();
            v.w = row + 3 < len ? __builtin_fmaf(cneg, acc[4 * g + 3], rn + xs[4 * g + 3]) : f_inf();
            *reinterpret_cast<float4*>(a.bufA + (uint64_t)q * a.capA + o + row) = v;
          }
        }
      }
    });
  });
}

// Stage B: every probed list against the query's bound.  Tiles and the
// ring as in stage A.
//   Test: s'_r = fma(-2^(1-er-xexp), acc_r, |x^_r|^2) <= T' with
//   T' = dkA + eps - |r|^2 rounded up: a code left out has s' > T', so its
//   screened distance exceeds dkA + eps by more than the FMA's rounding,
//   which eps covers.  The 16 values of a lane are reduced to their minimum
//   first; only lanes whose minimum passes form the row mask.  Rows past
//   the list's end have |x^|^2 = +inf, so s' = +inf; they are masked
//   explicitly only where T' is +inf.
//   Candidates: a lane with a passing row appends one 32-bit entry (row
//   mask | block in the chunk << 16 | lane << 24 | group << 30) to its wave's LDS queue
//   at the rank ballot and mbcnt give it: no atomics while blocks stream,
//   so the ring's loads stay in flight (an atomic with return waits for
//   every outstanding load).  At the end of the tile (or when the queue is
//   nearly full) each lane reserves its count in its query's candidate list
//   with one atomic, and the entries are written out.
// NS: stages of the ring; W: waves per SIMD the registers are sized for
// (measured at 1M x 128 codes, nprobe 16: NS 3 at 4 waves per SIMD 0.179 ms;
// NS 4 at 3 waves 0.186 ms; NS 6 and 8 at 2 waves 0.248 ms).  PG: groups
// of 32 pairs per wave (tiles of 128 PG pairs): with PG 2 a list chunk of up
// to 256 pairs is streamed through the ring once, each block multiplied
// against both groups' operands.
template <int KC, int NS, int W, int PG, int WV>
__global__ __launch_bounds__(64 * WV) __attribute__((amdgpu_waves_per_eu(W))) void pq16_thresh_kernel(ScreenArgs a) {
  static_assert(PG == 1 || PG == 2, "one or two groups of pairs per wave");
  constexpr uint32_t kQ = 256;  // queue entries per wave
  __shared__ Ring<KC, NS, WV> ring;
  __shared__ uint32_t wq[WV][kQ];
  __shared__ uint32_t wbase[WV][PG][64];  // each (group, lane)'s next position while flushing
  const int lane = threadIdx.x & 63;
  const int wave = wave_index();
  const int col = lane & 31;
  const int half = lane >> 5;
  __shared__ uint32_t s_next;
  const uint32_t ntiles = a.toff[a.nlist];
  for_tiles(ntiles, a.tctr, a.dyn, a.run, &s_next, [&](uint32_t t) {
    const TileWork w = tile_work<32 * WV * PG, WV>(a, t, wave);
    const uint32_t p = w.p;
    RingStream<KC, NS, WV> rs(ring, reinterpret_cast<const v4u*>(a.data) + (uint64_t)w.babs * KC * 64,
                              a.xnb + (uint64_t)w.babs * 32, w.nblk, wave, lane);
    rs.begin();
    const float X = sqrtf(__uint_as_float(a.xmax2[p])) * (1.0f + 0x1p-16f);
    uint32_t q[PG], j[PG];
    PairOperand<KC> op[PG];
    float Tp[PG], cneg[PG];
#pragma unroll
    for (int g = 0; g < PG; ++g) {
      const uint32_t qg = g == 0 ? w.q0 : w.q1;
      const bool gbusy = g == 0 ? w.busy : w.busy1;
      const bool qv = gbusy && qg + (uint32_t)col < w.qend;
      const uint2 e = a.qlist[min(qg + (uint32_t)col, w.qend - 1)];
      q[g] = e.x;
      j[g] = e.y;
      Tp[g] = -f_inf();  // no append
      cneg[g] = 0.0f;
      if (g > 0 && !gbusy) continue;  // wave-uniform
      pair_operand<KC>(a, q[g], p, half, op[g]);
      if (qv && op[g].bad && half == 0) atomicOr(&a.force[q[g]], 1);
      if (qv && !op[g].bad) {
        const float rnorm = sqrtf(op[g].rn) * (1.0f + 0x1p-16f);
        const float f = add_up(a.dkA[q[g]], pq16_eps(rnorm, X, a)) - op[g].rn;
        Tp[g] = f + __builtin_fabsf(f) * 0x1p-22f;
      }
      cneg[g] = -ldexpf(1.0f, 1 - op[g].er - a.xexp);
    }
    const uint32_t bb = w.babs - a.bo[p];  // the tile's first block in the list
    const uint32_t start = a.list_off[p];
    const uint32_t len = a.list_off[p + 1] - start;
    uint32_t* __restrict__ myq = wq[wave];
    uint32_t qn = 0;       // wave-uniform queue length
    uint32_t cnt[PG];      // this lane's entries in the queue, per group
#pragma unroll
    for (int g = 0; g < PG; ++g) cnt[g] = 0;
    // Queue to candidate list: one atomic per (lane, group) with entries
    // reserves its range; then 64 entries at a time, each lane takes one,
    // gets its slot from the owner's running position (an LDS atomic) and
    // writes (list position of the row base, probe index << 16 | mask).  All
    // lanes call this (the shuffles take every lane).
    auto flush = [&]() {
#pragma unroll
      for (int g = 0; g < PG; ++g) {
        wbase[wave][g][lane] = cnt[g] ? atomicAdd(&a.ccnt[q[g]], cnt[g]) : 0u;
        cnt[g] = 0;
      }
      __builtin_amdgcn_wave_barrier();
      for (uint32_t i0 = 0; i0 < qn; i0 += 64) {
        const uint32_t i = i0 + (uint32_t)lane;
        const uint32_t ent = i < qn ? myq[i] : 0u;
        const int owner = (int)((ent >> 24) & 63);
        const int g = PG > 1 ? (int)((ent >> 30) & 1) : 0;
        uint32_t oq = (uint32_t)__shfl((int)q[0], owner), oj = (uint32_t)__shfl((int)j[0], owner);
        if constexpr (PG > 1) {
          const uint32_t oq1 = (uint32_t)__shfl((int)q[PG - 1], owner), oj1 = (uint32_t)__shfl((int)j[PG - 1], owner);
          oq = g ? oq1 : oq;
          oj = g ? oj1 : oj;
        }
        if (i < qn) {
          const uint32_t pos = atomicAdd(&wbase[wave][g][owner], 1u);
          if (pos < a.cap) {
            const uint32_t rowb = (bb + ((ent >> 16) & 255)) * 32 + 4 * (uint32_t)(owner >> 5);
            a.cand[(uint64_t)oq * a.cap + pos] = make_uint2(start + rowb, (oj << 16) | (ent & 0xFFFFu));
          }
        }
      }
      qn = 0;
      __builtin_amdgcn_wave_barrier();
    };
    rs.run(w, [&](const v4u* __restrict__ sa, const float* __restrict__ sx, uint32_t sb) {
      const uint32_t b = bb + sb;
      // the block's k-chunks read once from LDS; with two groups each feeds
      // both groups' products (two independent chains)
      v4u av[KC];
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) av[kc] = sa[kc * 64 + lane];
      float xs[16];
      block_norms(sx, half, xs);
      const uint32_t rowb = b * 32 + 4 * half;
      v16f acc[PG];
#pragma unroll
      for (int g = 0; g < PG; ++g) acc[g] = v16f{};
      if (PG > 1 && w.busy1) {  // wave-uniform
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
#pragma unroll
          for (int g = 0; g < PG; ++g)
            acc[g] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, av[kc]), op[g].bq[kc], acc[g], 0,
                                                            0, 0);
      } else {
#pragma unroll
        for (int kc = 0; kc < KC; ++kc)
          acc[0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, av[kc]), op[0].bq[kc], acc[0], 0, 0,
                                                          0);
      }
#pragma unroll
      for (int g = 0; g < PG; ++g) {
        if (g > 0 && !w.busy1) break;  // wave-uniform
        float s[16];
#pragma unroll
        for (int rr = 0; rr < 16; ++rr) s[rr] = __builtin_fmaf(cneg[g], acc[g][rr], xs[rr]);
        const float m0 = fminf(fminf(s[0], s[1]), s[2]);
        const float m1 = fminf(fminf(s[3], s[4]), s[5]);
        const float m2 = fminf(fminf(s[6], s[7]), s[8]);
        const float m3 = fminf(fminf(s[9], s[10]), s[11]);
        const float m4 = fminf(fminf(s[12], s[13]), s[14]);
        const bool pass = fminf(fminf(fminf(m0, m1), fminf(m2, m3)), fminf(m4, s[15])) <= Tp[g];
        if (__ballot(pass) == 0) continue;
        uint32_t passm = 0;
        if (pass) {
#pragma unroll
          for (int rr = 0; rr < 16; ++rr) passm |= (s[rr] <= Tp[g] ? 1u : 0u) << rr;
          // rows past the list's end pass only a threshold of +inf
          if (rowb + 28 > len)
#pragma unroll
            for (int rr = 0; rr < 16; ++rr)
              if (rowb + 8 * (rr >> 2) + (rr & 3) >= len) passm &= ~(1u << rr);
        }
        // one entry per lane, group and block with a passing row: its
        // 16-row mask (rows 8(i/4) + i%4 from the lane's row base)
        const uint64_t bal = __ballot(passm != 0);
        if (bal == 0) continue;
        if (passm != 0) {
          const uint32_t rank =
              __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
          myq[qn + rank] = passm | ((b - bb) << 16) | ((uint32_t)lane << 24) | ((uint32_t)g << 30);
          ++cnt[g];
        }
        qn += (uint32_t)__popcll(bal);
        if (qn > kQ - 64) flush();
      }
    });
    if (qn > 0) flush();
  });
}

// Stage B's kernel for KC k-chunks
template <int KC>
void (*thresh_kernel())(ScreenArgs) {
  return pq16_thresh_kernel<KC, stage_b_stages(KC), stage_b_waves(KC), stage_b_groups(KC), stage_b_wgwaves(KC)>;
}

// One wave per query: dkA = (k-th smallest kept screened value) + the
// largest bound among its first lists, rounded up: at least k codes of
// those lists have reference distance <= dkA, so the final k-th does too.
// +inf when fewer than k codes were kept (the padding holds +inf).
template <int R>
__global__ __launch_bounds__(64) void pq16_select_kernel(const float* __restrict__ bufA, uint32_t capA,
                                                         const uint32_t* __restrict__ nA,
                                                         const uint32_t* __restrict__ nreal,
                                                         const uint32_t* __restrict__ jlim,
                                                         const float* __restrict__ epsA, int np, int k,
                                                         int margin, float* __restrict__ dkA) {
  __shared__ uint2 queue[64];
  const uint64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  const uint32_t n = nA[q];
  if (nreal[q] < (uint32_t)k) {
    if (lane == 0) dkA[q] = f_inf();
    return;
  }
  WaveTopK<R> tk;
  tk.init(k);
  int qn = 0;
  // (a plain vector type: loop-carried HIP float4 values can end up in
  // scratch memory)
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4* __restrict__ v = reinterpret_cast<const f4*>(bufA + q * capA);
  const uint32_t n4 = (n + 3) / 4;  // n is a multiple of 32 or capA
  const f4 none = {f_inf(), f_inf(), f_inf(), f_inf()};
  // k <= 64 (k <= 128): each lane's smallest value (four smallest) goes in
  // first; the k-th smallest of those bounds the k-th overall, so that few of
  // the others get past the list's threshold (one merge instead of one per
  // 64 early values, and few insertions after it).  Every value is offered
  // once either way.
  constexpr int S = R == 1 ? 1 : (R == 2 ? 4 : 0);  // seeds per lane
  uint32_t si[S > 0 ? S : 1];
#pragma unroll
  for (int j = 0; j < (S > 0 ? S : 1); ++j) si[j] = kNoPos;
  if constexpr (S > 0) {
    float ms[S];
#pragma unroll
    for (int j = 0; j < S; ++j) ms[j] = f_inf();
    // sorted insertion of (x, i) into the lane's S smallest
    auto seed = [&](float x, uint32_t i) {
#pragma unroll
      for (int j = S - 1; j > 0; --j) {
        if (x < ms[j - 1]) {
          ms[j] = ms[j - 1];
          si[j] = si[j - 1];
        } else if (x < ms[j]) {
          ms[j] = x;
          si[j] = i;
        }
      }
      if (x < ms[0]) {
        ms[0] = x;
        si[0] = i;
      }
    };
#pragma unroll 1
    for (uint32_t i0 = 0; i0 < n4; i0 += 64) {
      const uint32_t il = i0 + (uint32_t)lane;
      const f4 w = il < n4 ? v[il] : none;
      const uint32_t i = 4 * il;
      seed(w.x, i);
      seed(w.y, i + 1);
      seed(w.z, i + 2);
      seed(w.w, i + 3);
    }
#pragma unroll
    for (int j = 0; j < S; ++j) tk.offer_queued(ms[j], si[j], ms[j] < f_inf(), queue, qn);
    tk.flush(queue, qn);
  }
  auto seeded = [&](uint32_t i) {
    bool r = false;
#pragma unroll
    for (int j = 0; j < (S > 0 ? S : 1); ++j) r = r || i == si[j];
    return r;
  };
  f4 w = (uint32_t)lane < n4 ? v[lane] : none;
#pragma unroll 1
  for (uint32_t i0 = 0; i0 < n4; i0 += 64) {
    const uint32_t inext = i0 + 64 + (uint32_t)lane;
    const f4 wn = inext < n4 ? v[inext] : none;  // the next values in flight
    const uint32_t i = 4 * (i0 + (uint32_t)lane);
    tk.offer_queued(w.x, i, w.x < f_inf() && !seeded(i), queue, qn);
    tk.offer_queued(w.y, i + 1, w.y < f_inf() && !seeded(i + 1), queue, qn);
    tk.offer_queued(w.z, i + 2, w.z < f_inf() && !seeded(i + 2), queue, qn);
    tk.offer_queued(w.w, i + 3, w.w < f_inf() && !seeded(i + 3), queue, qn);
    w = wn;
  }
  tk.flush(queue, qn);
  float em = 0.0f;
  for (uint32_t j = 0; j < jlim[q]; ++j) em = fmaxf(em, epsA[q * np + j]);
  if (lane == 0) {
    // margin (the Euclidean metric): rows whose square roots tie with the
    // k-th's may exceed its squared distance by a few ulps
    const float dk = add_up(tk.tau, em);
    dkA[q] = margin ? dk + __builtin_fabsf(dk) * 0x1p-20f : dk;
  }
}

// ---- exact rescoring ----------------------------------------------------------

// One table entry of the reference (l2sq_ref order on r - cb, r = q - c)
// computed from the query, centroid and codeword rows of one subspace.
__device__ __forceinline__ float pq_entry(const float* __restrict__ qs, const float* __restrict__ cen,
                                          const float* __restrict__ cw, int dsub) {
  const int nb = dsub / 8;
  float total = 0.0f;
  if (nb > 0) {
    float lane[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) lane[l] = 0.0f;
    for (int i = 0; i < nb; ++i)
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const float r = qs[8 * i + l] - cen[8 * i + l];
        const float d = r - cw[8 * i + l];
        lane[l] = __builtin_fmaf(d, d, lane[l]);
      }
    total = lane[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) total = total + lane[l];
  }
  for (int i = 8 * nb; i < dsub; ++i) {
    const float r = qs[i] - cen[i];
    const float d = r - cw[i];
    total = total + d * d;
  }
  return total;
}

struct RescoreArgs16 {
  const float* queries;
  int D, M, dsub;
  const int32_t* probes;
  int np;
  const float* centroids;
  const float* codebooks;
  const float* cb4;  // codebooks with codewords padded to a multiple of 4 floats
  int nlist;
  int cached;        // residuals of every probe in LDS
  const uint8_t* codes;
  const uint64_t* ids;
  const uint32_t* ccnt;
  const uint2* cand;
  uint32_t cap;
  const int* force;
  int k, order;
  const float* rows;  // full vectors in list order (Pq16SearchArgs::rows), or null
  int sqrt_out;       // with rows: the square root of the squared L2 (Euclidean)
  uint64_t* out_ids;
  float* out_d;
  uint32_t* out_counts;
  int* flags;
  uint32_t* nexp;    // [nq] candidates of each entry list, expanded (statistics)
  const uint2* heavy;        // parts of the queries of more than kLight entries:
                             // (query, part | parts << 16), or (~0, 0) for none
  uint32_t pmax;             // part slots
  float* part_d;             // [pmax][k] each part's list, when a query has several
  uint32_t* part_k;
  const uint32_t* qorder;    // the other queries: counters[1] at the front, counters[2] at the back
  const uint32_t* counters;  // pq16_classify_kernel's
};

// The row offset, from an entry's row base, of the lowest set bit i of its
// mask: 8(i/4) + i%4 (the MFMA output layout of the lane's 16 rows).
__device__ __forceinline__ uint32_t entry_row(uint32_t mask) {
  const uint32_t i = (uint32_t)__ffs(mask) - 1u;
  return 8u * (i >> 2) + (i & 3u);
}

// Expands one wave's batch of entries (lane l: entry e, valid v) into its
// candidates, 64 per round: f(has, key, probe index) is called by every lane
// each round, has false past the last candidate.  ent and pre: the wave's
// 64-entry LDS arrays.
template <class F>
__device__ __forceinline__ void expand_entries(uint2 e, bool v, uint2* ent, uint32_t* pre, F&& f) {
  const int lane = threadIdx.x & 63;
  const uint32_t n = v ? (uint32_t)__popc(e.y & 0xFFFFu) : 0u;
  uint32_t x = n;  // inclusive prefix over the lanes
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const uint32_t y = (uint32_t)__shfl_up((int)x, off);
    if (lane >= off) x += y;
  }
  const uint32_t total = (uint32_t)__shfl((int)x, 63);
  if (total == (uint32_t)__popcll(__ballot(v))) {  // one row per entry (the usual case)
    f(v, v ? e.x + entry_row(e.y & 0xFFFFu) : kNoPos, e.y >> 16);
    return;
  }
  ent[lane] = e;
  pre[lane] = x;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (uint32_t r0 = 0; r0 < total; r0 += 64) {
    const uint32_t t = r0 + (uint32_t)lane;
    const bool has = t < total;
    uint32_t key = kNoPos, jj = 0;
    if (has) {
      uint32_t lo = 0, hi = 63;  // the first entry whose inclusive prefix exceeds t
      while (lo < hi) {
        const uint32_t mid = (lo + hi) >> 1;
        if (pre[mid] > t) hi = mid;
        else lo = mid + 1;
      }
      const uint2 en = ent[lo];
      uint32_t m = en.y & 0xFFFFu;
      for (uint32_t rank = t - (lo ? pre[lo - 1] : 0u); rank > 0; --rank) m &= m - 1;
      key = en.x + entry_row(m);
      jj = en.y >> 16;
    }
    f(has, key, jj);
  }
  __builtin_amdgcn_wave_barrier();  // ent and pre are rewritten by the next batch
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off);
  return v;
}

// One table entry from the cached residual row r of the subspace (LDS) and
// the codeword cw (padded to a multiple of 4 floats): the l2sq_ref order on
// r - cw.  DS: dsub at compile time (0 = runtime).
template <int DS>
__device__ __forceinline__ float entry_cached(const float* __restrict__ r, const float* __restrict__ cw, int dsub) {
  if constexpr (DS > 0) {
    constexpr int DS4 = (DS + 3) / 4 * 4;
    float c[DS4];
#pragma unroll
    for (int i = 0; i < DS4 / 4; ++i) {
      const float4 v = reinterpret_cast<const float4*>(cw)[i];
      c[4 * i] = v.x;
      c[4 * i + 1] = v.y;
      c[4 * i + 2] = v.z;
      c[4 * i + 3] = v.w;
    }
    constexpr int NB = DS / 8;
    float total = 0.0f;
    if constexpr (NB > 0) {
      float lane[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const float d = r[l] - c[l];
        lane[l] = __builtin_fmaf(d, d, 0.0f);
      }
#pragma unroll
      for (int i = 1; i < NB; ++i)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const float d = r[8 * i + l] - c[8 * i + l];
          lane[l] = __builtin_fmaf(d, d, lane[l]);
        }
      total = lane[0];
#pragma unroll
      for (int l = 1; l < 8; ++l) total = total + lane[l];
    }
#pragma unroll
    for (int i = 8 * NB; i < DS; ++i) {
      const float d = r[i] - c[i];
      total = total + d * d;
    }
    return total;
  } else {
    const int nb = dsub / 8;
    float total = 0.0f;
    if (nb > 0) {
      float lane[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) lane[l] = 0.0f;
      for (int i = 0; i < nb; ++i)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const float d = r[8 * i + l] - cw[8 * i + l];
          lane[l] = __builtin_fmaf(d, d, lane[l]);
        }
      total = lane[0];
#pragma unroll
      for (int l = 1; l < 8; ++l) total = total + lane[l];
    }
    for (int i = 8 * nb; i < dsub; ++i) {
      const float d = r[i] - cw[i];
      total = total + d * d;
    }
    return total;
  }
}

// The reference's squared L2 (euclidean_distance_squared_avx2,
// src/distance/simd.rs:335-366: 8 FMA lanes over the 8-float chunks, the
// lanes summed 0..7, a scalar tail) of a query in LDS and a row in global
// memory; with a row length a multiple of 4, the row is read 16 bytes at a
// time, 16 loads in flight.
__device__ __forceinline__ float row_l2sq(const float* __restrict__ q, const float* __restrict__ x, int n) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const int nb = n / 8;
  float total = 0.0f;
  if (nb > 0) {
    float l[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) l[t] = 0.0f;
    if ((n & 3) == 0) {
      const f4* __restrict__ x4 = reinterpret_cast<const f4*>(x);
      for (int i0 = 0; i0 < nb; i0 += 8) {
        f4 v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (2 * i0 + j < 2 * nb) v[j] = x4[2 * i0 + j];
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (i0 + j < nb) {
            const float* __restrict__ qi = q + 8 * (i0 + j);
#pragma unroll
            for (int t = 0; t < 8; ++t) {
              const float d = qi[t] - (t < 4 ? v[2 * j][t] : v[2 * j + 1][t - 4]);
              l[t] = __builtin_fmaf(d, d, l[t]);
            }
          }
      }
    } else {
      for (int i = 0; i < nb; ++i)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = q[8 * i + t] - x[8 * i + t];
          l[t] = __builtin_fmaf(d, d, l[t]);
        }
    }
    total = l[0];
#pragma unroll
    for (int t = 1; t < 8; ++t) total = total + l[t];
  }
  for (int i = 8 * nb; i < n; ++i) {
    const float d = q[i] - x[i];
    total = total + d * d;
  }
  return total;
}

// The exact distance of a full-vector candidate (list position key).
__device__ __forceinline__ float row_dist(const RescoreArgs16& a, const float* __restrict__ qs, uint32_t key) {
  const float t = row_l2sq(qs, a.rows + (uint64_t)key * a.D, a.D);
  return a.sqrt_out ? __builtin_sqrtf(t) : t;
}

// The reference's distance of one code: entries v(m) summed in adc_sum order.
template <class V>
__device__ __forceinline__ float adc_order(int M, int order, V v) {
  if (order == kAdcLanes8) {
    const int mb = M / 8;
    float total = 0.0f;
    if (mb > 0) {
      float lane[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) lane[l] = v(l);
#pragma unroll
      for (int b = 1; b < mb; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) lane[l] = lane[l] + v(8 * b + l);
      total = lane[0];
#pragma unroll
      for (int l = 1; l < 8; ++l) total = total + lane[l];
    }
    for (int m = 8 * mb; m < M; ++m) total = total + v(m);
    return total;
  }
  float sum = 0.0f;
  int m = 0;
#pragma unroll
  for (; m + 4 <= M; m += 4) {
    float t = v(m) + v(m + 1);
    t = t + v(m + 2);
    t = t + v(m + 3);
    sum = sum + t;
  }
  for (; m < M; ++m) sum = sum + v(m);
  return sum;
}

// A candidate's code row: MM (a multiple of 16, at compile time) bytes read
// as 16-byte words, else byte by byte from the row.
template <int MM>
struct CodeRow {
  uint32_t w[MM > 0 ? MM / 4 : 1];
  const uint8_t* row;
  __device__ __forceinline__ CodeRow(const uint8_t* r) : row(r) {
    if constexpr (MM > 0) {
#pragma unroll
      for (int i = 0; i < MM / 16; ++i) {
        const uint4 v = reinterpret_cast<const uint4*>(r)[i];
        w[4 * i] = v.x;
        w[4 * i + 1] = v.y;
        w[4 * i + 2] = v.z;
        w[4 * i + 3] = v.w;
      }
    }
  }
  __device__ __forceinline__ uint32_t operator[](int m) const {
    if constexpr (MM > 0) return (w[m >> 2] >> (8 * (m & 3))) & 0xFFu;
    else return row[m];
  }
};

// One table entry from the query (LDS), centroid and padded codeword rows
// of one subspace, the l2sq_ref order on (q - c) - cw; DS: dsub at compile
// time (0 = runtime), 16-byte loads where the rows allow.
template <int DS>
__device__ __forceinline__ float entry_direct(const float* __restrict__ qs, const float* __restrict__ cen,
                                             const float* __restrict__ cw, int dsub) {
  if constexpr (DS > 0) {
    constexpr int DS4 = (DS + 3) / 4 * 4;
    float c[DS4], cn[DS];
#pragma unroll
    for (int i = 0; i < DS4 / 4; ++i) {
      const float4 v = reinterpret_cast<const float4*>(cw)[i];
      c[4 * i] = v.x;
      c[4 * i + 1] = v.y;
      c[4 * i + 2] = v.z;
      c[4 * i + 3] = v.w;
    }
    if constexpr (DS % 4 == 0) {
#pragma unroll
      for (int i = 0; i < DS / 4; ++i) {
        const float4 v = reinterpret_cast<const float4*>(cen)[i];
        cn[4 * i] = v.x;
        cn[4 * i + 1] = v.y;
        cn[4 * i + 2] = v.z;
        cn[4 * i + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < DS; ++i) cn[i] = cen[i];
    }
    constexpr int NB = DS / 8;
    float total = 0.0f;
    if constexpr (NB > 0) {
      float lane[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        const float d = (qs[l] - cn[l]) - c[l];
        lane[l] = __builtin_fmaf(d, d, 0.0f);
      }
#pragma unroll
      for (int i = 1; i < NB; ++i)
#pragma unroll
        for (int l = 0; l < 8; ++l) {
          const float d = (qs[8 * i + l] - cn[8 * i + l]) - c[8 * i + l];
          lane[l] = __builtin_fmaf(d, d, lane[l]);
        }
      total = lane[0];
#pragma unroll
      for (int l = 1; l < 8; ++l) total = total + lane[l];
    }
#pragma unroll
    for (int i = 8 * NB; i < DS; ++i) {
      const float d = (qs[i] - cn[i]) - c[i];
      total = total + d * d;
    }
    return total;
  } else {
    return pq_entry(qs, cen, cw, dsub);
  }
}

// Thread per query: its flag (1: table scan, for a residual out of fp16
// range or more candidate entries than slots) and its place in the
// rescoring: more than kLight entries, ceil(entries / kPart) parts in the
// heavy list (a workgroup each; multi-part queries also in multi as (query,
// first part), merged afterwards); more than kRound, the front of order;
// else its back (filled from the end), so that the longer lists start
// first.  counters: [0] heavy parts, [1] front, [2] back, [3] multi.  A
// query whose parts do not fit the pmax part slots is flagged.
__global__ __launch_bounds__(kT) void pq16_classify_kernel(const uint32_t* __restrict__ ccnt,
                                                           const int* __restrict__ force, uint32_t cap,
                                                           uint64_t nq, int* __restrict__ flags,
                                                           uint32_t* __restrict__ order,
                                                           uint2* __restrict__ heavy, uint32_t pmax,
                                                           uint2* __restrict__ multi,
                                                           uint32_t* __restrict__ nexp,
                                                           uint32_t* __restrict__ counters) {
  const uint64_t q = (uint64_t)blockIdx.x * kT + threadIdx.x;
  const int lane = threadIdx.x & 63;
  const bool valid = q < nq;
  const uint32_t cnt = valid ? ccnt[q] : 0u;
  bool fall = valid && (force[q] != 0 || cnt > cap);
  if (valid && !fall && cnt > kLight) {
    const uint32_t parts = (cnt + kPart - 1) / kPart;
    const uint32_t base = atomicAdd(&counters[0], parts);
    if (base + parts <= pmax) {
      for (uint32_t i = 0; i < parts; ++i) heavy[base + i] = make_uint2((uint32_t)q, i | (parts << 16));
      multi[atomicAdd(&counters[3], 1u)] = make_uint2((uint32_t)q, base);
      nexp[q] = 0;  // the parts add theirs
    } else {
      for (uint32_t i = base; i < min(base + parts, pmax); ++i) heavy[i] = make_uint2(~0u, 0u);
      fall = true;
    }
  }
  if (valid) flags[q] = fall ? 1 : 0;
  const int cls = (!valid || fall) ? -1 : (cnt > kLight ? 0 : (cnt > kRound ? 1 : 2));
#pragma unroll
  for (int c = 1; c < 3; ++c) {
    const uint64_t m = __ballot(cls == c);
    if (m == 0) continue;
    const int leader = __ffsll((long long)m) - 1;
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(&counters[c], (uint32_t)__popcll(m));
    base = (uint32_t)__shfl((int)base, leader);
    const uint32_t rank = __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (cls == c) {
      if (c == 1) order[base + rank] = (uint32_t)q;
      else order[nq - 1 - (base + rank)] = (uint32_t)q;
    }
  }
}

// One wave per query (have: the wave has one): a query of at most kLight
// candidate entries scored and selected as in pq16_rescore_heavy.  Every wave
// of the workgroup calls it (one workgroup barrier).
template <int R, int DS, int MM>
__device__ __forceinline__ void pq16_rescore_light(const RescoreArgs16& a, uint64_t q, bool have) {
  __shared__ float qsm[kT / 64][256];
  __shared__ uint2 queue[kT / 64][64];
  __shared__ uint2 xent[kT / 64][64];
  __shared__ uint32_t xpre[kT / 64][64];
  const int lane = threadIdx.x & 63;
  const int wave = wave_index();
  const uint32_t cnt = have ? a.ccnt[q] : 0u;
  const int D = a.D;
  if (have)
    for (int d = lane; d < D; d += 64) qsm[wave][d] = a.queries[q * D + d];
  __syncthreads();
  if (!have) return;
  const float* __restrict__ qs = qsm[wave];
  WaveTopK<R> tk;
  tk.init(a.k);
  int qn = 0;
  const uint2* __restrict__ cq = a.cand + q * a.cap;
  const int M = MM > 0 ? MM : a.M, dsub = DS > 0 ? DS : a.dsub;
  const int ds4 = (dsub + 3) / 4 * 4;
  uint32_t ncand = 0;
  for (uint32_t c0 = 0; c0 < cnt; c0 += 64) {
    const uint32_t c = c0 + (uint32_t)lane;
    const uint2 e = c < cnt ? cq[c] : make_uint2(0u, 0u);
    expand_entries(e, c < cnt, xent[wave], xpre[wave], [&](bool has, uint32_t key, uint32_t jj) {
      float d = f_inf();
      if (has) {
        ++ncand;
        if constexpr (DS < 0) {
          d = row_dist(a, qs, key);
        } else {
          const CodeRow<MM> code(a.codes + (uint64_t)key * M);
          const float* __restrict__ cen = a.centroids + (uint64_t)a.probes[q * a.np + jj] * D;
          d = adc_order(M, a.order, [&](int m) {
            return entry_direct<DS>(qs + m * dsub, cen + m * dsub, a.cb4 + ((uint64_t)m * 256 + code[m]) * ds4,
                                    dsub);
          });
        }
      }
      tk.offer_queued(d, key, has, queue[wave], qn);
    });
  }
  tk.flush(queue[wave], qn);
  ncand = wave_sum(ncand);
  if (lane == 0) a.nexp[q] = ncand;
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = r * 64 + lane;
    const bool valid = s < a.k && tk.p[r] != kNoPos;
    count += (uint32_t)__popcll(__ballot(valid));
    if (s < a.k) {
      a.out_ids[q * a.k + s] = valid ? a.ids[tk.p[r]] : ~0ull;
      a.out_d[q * a.k + s] = valid ? tk.d[r] : f_inf();
    }
  }
  if (lane == 0) a.out_counts[q] = count;
}

// Four waves per query: the candidates' reference distances (wave w takes
// every fourth batch of 64) and the top k (ties: smaller list position, as
// the table scan), the wave lists merged by wave 0.  The residuals r_j =
// q - c_(probe j) are computed once into LDS (rc [np][D]) when they fit
// (cached), else per candidate.  Queries with a residual out of fp16 range
// or more candidates than slots are flagged for the table scan.
// Part `part` of `parts` (entries [part*kPart, +kPart)) of a query of more
// than kLight candidate entries, by the whole workgroup; its list goes to
// part slot `slot` for pq16_merge_kernel.
template <int R, int DS, int MM>
__device__ __forceinline__ void pq16_rescore_heavy(RescoreArgs16 a, uint64_t q, uint32_t part, uint32_t parts,
                                                   uint32_t slot) {
  extern __shared__ float qs[];  // [D], then rc [np][D] when cached
  __shared__ uint2 queue[kT / 64][64];
  __shared__ float md[kT / 64][64 * R];
  __shared__ uint32_t mk[kT / 64][64 * R];
  __shared__ uint32_t nsum[kT / 64];
  __shared__ uint2 xent[kT / 64][64];
  __shared__ uint32_t xpre[kT / 64][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t e0 = part * kPart, cnt = min(a.ccnt[q], e0 + kPart);
  const int D = a.D;
  float* rc = qs + D;
  // a few candidates are cheaper to rescore without the residual cache
  const bool cached = a.cached && cnt - e0 >= 128;
  for (int d = tid; d < D; d += kT) qs[d] = a.queries[q * D + d];
  if (cached) {
    for (int e = tid; e < a.np * D; e += kT) {
      const int j = e / D;
      const int d = e - j * D;
      const int32_t p = a.probes[q * a.np + j];
      rc[e] = (p >= 0 && p < a.nlist) ? a.queries[q * D + d] - a.centroids[(uint64_t)p * D + d] : 0.0f;
    }
  }
  __syncthreads();
  WaveTopK<R> tk;
  tk.init(a.k);
  int qn = 0;
  const uint2* __restrict__ cq = a.cand + q * a.cap;
  const int M = MM > 0 ? MM : a.M, dsub = DS > 0 ? DS : a.dsub;
  const int ds4 = (dsub + 3) / 4 * 4;
  uint32_t ncand = 0;
  for (uint32_t c0 = e0 + (uint32_t)wave * 64; c0 < cnt; c0 += kT) {
    const uint32_t c = c0 + (uint32_t)lane;
    const uint2 e = c < cnt ? cq[c] : make_uint2(0u, 0u);
    expand_entries(e, c < cnt, xent[wave], xpre[wave], [&](bool has, uint32_t key, uint32_t jj) {
      float d = f_inf();
      if constexpr (DS < 0) {
        if (has) {
          ++ncand;
          d = row_dist(a, qs, key);
        }
      } else if (has) {
        ++ncand;
        const CodeRow<MM> code(a.codes + (uint64_t)key * M);
        if (cached) {
          const float* __restrict__ rr = rc + jj * D;
          d = adc_order(M, a.order, [&](int m) {
            return entry_cached<DS>(rr + m * dsub, a.cb4 + ((uint64_t)m * 256 + code[m]) * ds4, dsub);
          });
        } else {
          const float* __restrict__ cen = a.centroids + (uint64_t)a.probes[q * a.np + jj] * D;
          d = adc_order(M, a.order, [&](int m) {
            return pq_entry(qs + m * dsub, cen + m * dsub, a.codebooks + ((uint64_t)m * 256 + code[m]) * dsub,
                            dsub);
          });
        }
      }
      tk.offer_queued(d, key, has, queue[wave], qn);
    });
  }
  tk.flush(queue[wave], qn);
  ncand = wave_sum(ncand);
  if (lane == 0) nsum[wave] = ncand;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    md[wave][r * 64 + lane] = tk.d[r];
    mk[wave][r * 64 + lane] = tk.p[r];
  }
  __syncthreads();
  if (wave != 0) return;  // waves 1-3 go on to the caller's barrier
  if (lane == 0) atomicAdd(&a.nexp[q], nsum[0] + nsum[1] + nsum[2] + nsum[3]);
  for (int w = 1; w < kT / 64; ++w)
#pragma unroll
    for (int r = 0; r < R; ++r) tk.offer(md[w][r * 64 + lane], mk[w][r * 64 + lane]);
  if (parts > 1) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int s = r * 64 + lane;
      if (s < a.k) {
        a.part_d[(uint64_t)slot * a.k + s] = tk.d[r];
        a.part_k[(uint64_t)slot * a.k + s] = tk.p[r];
      }
    }
    return;
  }
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = r * 64 + lane;
    const bool valid = s < a.k && tk.p[r] != kNoPos;
    count += (uint32_t)__popcll(__ballot(valid));
    if (s < a.k) {
      a.out_ids[q * a.k + s] = valid ? a.ids[tk.p[r]] : ~0ull;
      a.out_d[q * a.k + s] = valid ? tk.d[r] : f_inf();
    }
  }
  if (lane == 0) a.out_counts[q] = count;
}

// Workgroups [0, nh) take the heavy list, one query at a time; the others
// four queries of order each, the longer lists (front) dispatched first.
// Registers for two waves per SIMD: the candidates' codeword and centroid
// gathers stay in flight together (measured 97 against 107 us at 1M x 128,
// 446 against 488 us at 10M x 96, with three waves per SIMD).
template <int R, int DS, int MM>
__global__ __launch_bounds__(kT) __attribute__((amdgpu_waves_per_eu(2))) void pq16_rescore_kernel(RescoreArgs16 a,
                                                                                                   uint64_t nq,
                                                                                                   uint32_t nh) {
  if (blockIdx.x < nh) {
    const uint32_t nparts = min(a.counters[0], a.pmax);
    for (uint32_t h = blockIdx.x; h < nparts; h += nh) {
      const uint2 it = a.heavy[h];
      if (it.x == ~0u) continue;  // a query whose parts did not fit (flagged)
      pq16_rescore_heavy<R, DS, MM>(a, it.x, it.y & 0xFFFFu, it.y >> 16, h);
      __syncthreads();  // the LDS is reused by the next part
    }
    return;
  }
  const uint64_t i = (uint64_t)(blockIdx.x - nh) * (kT / 64) + wave_index();
  const uint32_t nf = a.counters[1], nb = a.counters[2];
  const bool have = i < nq && (i < nf || i >= nq - nb);
  pq16_rescore_light<R, DS, MM>(a, have ? a.qorder[i] : 0, have);
}

// Waves per query of pq16_merge_kernel: four for lists of more than 64
// (at 10M x 96, k 100, the merge took 56 instead of 98 us), one for the
// shorter ones (7 against 8 us at 1M x 128, k 10, where few queries have
// several parts).
constexpr int merge_waves(int R) { return R >= 2 ? 4 : 1; }

// A workgroup of NW waves per query of several parts (multi [counters[3]]:
// query, first part slot): wave w merges the lists of parts w, w + NW, ...
// by (distance, list position), then wave 0 merges the NW lists, which
// selects what one pass over every entry would.
template <int R, int NW>
__global__ __launch_bounds__(64 * NW) void pq16_merge_kernel(RescoreArgs16 a, const uint2* __restrict__ multi) {
  __shared__ uint2 queue[NW][64];
  __shared__ float md[NW][64 * R];
  __shared__ uint32_t mk[NW][64 * R];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (uint32_t m = blockIdx.x; m < a.counters[3]; m += gridDim.x) {
    const uint2 mq = multi[m];
    const uint64_t q = mq.x;
    const uint32_t parts = (a.ccnt[q] + kPart - 1) / kPart;
    WaveTopK<R> tk;
    tk.init(a.k);
    int qn = 0;
    for (uint32_t pt = (uint32_t)wave; pt < parts; pt += NW)
      for (int r0 = 0; r0 < a.k; r0 += 64) {
        const int s = r0 + lane;
        const uint64_t i = (uint64_t)(mq.y + pt) * a.k + s;
        const uint32_t key = s < a.k ? a.part_k[i] : kNoPos;
        const bool valid = key != kNoPos;
        tk.offer_queued(valid ? a.part_d[i] : f_inf(), key, valid, queue[wave], qn);
      }
    tk.flush(queue[wave], qn);
    if constexpr (NW > 1) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        md[wave][r * 64 + lane] = tk.d[r];
        mk[wave][r * 64 + lane] = tk.p[r];
      }
      __syncthreads();
    }
    if (wave == 0) {
      for (int w = 1; w < NW; ++w)
#pragma unroll
        for (int r = 0; r < R; ++r) tk.offer(md[w][r * 64 + lane], mk[w][r * 64 + lane]);
      uint32_t count = 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int s = r * 64 + lane;
        const bool valid = s < a.k && tk.p[r] != kNoPos;
        count += (uint32_t)__popcll(__ballot(valid));
        if (s < a.k) {
          a.out_ids[q * a.k + s] = valid ? a.ids[tk.p[r]] : ~0ull;
          a.out_d[q * a.k + s] = valid ? tk.d[r] : f_inf();
        }
      }
      if (lane == 0) a.out_counts[q] = count;
    }
    if constexpr (NW > 1) __syncthreads();  // md, mk and the queues are rewritten for the next query
  }
}

// One workgroup: stat[0] += queries flagged, stat[2..3] += expanded
// candidates (ncand) of the others (= with clear).
__global__ __launch_bounds__(1024) void pq16_stats_kernel(const int* __restrict__ flags,
                                                          const uint32_t* __restrict__ ncand, uint64_t nq,
                                                          int clear, uint32_t* __restrict__ stat) {
  __shared__ unsigned long long red[2][16];
  unsigned long long f = 0, c = 0;
  for (uint64_t q = threadIdx.x; q < nq; q += 1024) {
    if (flags[q]) f += 1;
    else c += ncand[q];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    f += __shfl_xor(f, off);
    c += __shfl_xor(c, off);
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[0][wave] = f;
    red[1][wave] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 16; ++w) {
      f += red[0][w];
      c += red[1][w];
    }
    if (clear) {
      stat[0] = (uint32_t)f;
      *reinterpret_cast<unsigned long long*>(&stat[2]) = c;
    } else {
      stat[0] += (uint32_t)f;
      *reinterpret_cast<unsigned long long*>(&stat[2]) += c;
    }
  }
}

// Bound coefficients (screen_eps_coeffs) for a reference distance whose
// terms are each rounded at most nref times (Pq16Lists::nref).
void pq16_eps_coeffs(int D16, int nref, float cmax, float& c_dot, float& c_sq, float& cabs) {
  screen_eps_coeffs(D16, nref, cmax, c_dot, c_sq, cabs);
}

}  // namespace

void Pq16Lists::build(const float* d_codebooks, const uint8_t* d_codes, const uint32_t* d_off,
                      const std::vector<uint64_t>& offsets, uint32_t nl, int m, int ds, hipStream_t s) {
  ok = false;
  M = m;
  dsub = ds;
  D = M * dsub;
  KC = (D + 15) / 16;
  nlist = nl;
  // the reference's table distance sums M entries, each a sum of dsub
  // squares of differences: a term is rounded at most dsub + M + 2 times
  // (the residual's and the difference's subtractions included)
  nref = dsub + M + 2;
  // B operands beyond 64 registers, or lists beyond the LDS counting sort:
  // the table scan only
  if (KC > 16 || nlist == 0 || nlist > kHistMax) return;
  std::vector<uint32_t> hbo(nlist + 1, 0);
  uint64_t nbk = 0;
  max_blocks = 0;
  for (uint32_t p = 0; p < nlist; ++p) {
    hbo[p] = (uint32_t)nbk;
    const uint64_t nb = cdiv(offsets[p + 1] - offsets[p], 32);
    nbk += nb;
    max_blocks = std::max(max_blocks, nb);
  }
  if (nbk >= 0xFFFFFFFFull) return;
  hbo[nlist] = (uint32_t)nbk;
  nblocks = nbk;
  bo.upload(hbo.data(), hbo.size(), s);
  stats.reserve(1);
  hipLaunchKernelGGL(pq16_fill_u32, dim3(1), dim3(kT), 0, s, stats.p, (uint64_t)1, 0u);
  FDB_HIP(hipGetLastError());
  const uint64_t ncb = (uint64_t)M * 256 * dsub;
  hipLaunchKernelGGL(pq16_cb_stats_kernel, dim3((unsigned)std::min<uint64_t>(cdiv(ncb, kT), 1024)), dim3(kT), 0, s,
                     d_codebooks, ncb, stats.p);
  FDB_HIP(hipGetLastError());
  uint32_t mbits = 0;
  FDB_HIP(hipMemcpyAsync(&mbits, stats.p, 4, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  if (mbits >= 0x7F800000u) return;  // a non-finite codebook component
  float mxv;
  std::memcpy(&mxv, &mbits, 4);
  cmax = mxv;
  xexp = 0;
  if (mxv > 0.0f) {
    int E;
    (void)std::frexp(mxv, &E);
    xexp = 13 - E;
  }
  if (xexp > 100 || xexp < -100) return;
  const int ds4 = (dsub + 3) / 4 * 4;
  cb4.reserve((uint64_t)M * 256 * ds4);
  hipLaunchKernelGGL(pq16_pad_cb_kernel, dim3((unsigned)cdiv((uint64_t)M * 256 * ds4, kT)), dim3(kT), 0, s,
                     d_codebooks, (uint64_t)M * 256, dsub, ds4, cb4.p);
  FDB_HIP(hipGetLastError());
  data.reserve(std::max<uint64_t>(nblocks * KC * 64, 1));
  xnb.reserve(std::max<uint64_t>(nblocks * 32, 1));
  xmax2.reserve(nlist);
  hipLaunchKernelGGL(pq16_fill_u32, dim3((unsigned)std::min<uint64_t>(cdiv(nlist, kT), 1024)), dim3(kT), 0, s,
                     xmax2.p, (uint64_t)nlist, 0u);
  FDB_HIP(hipGetLastError());
  if (nblocks > 0) {
    hipLaunchKernelGGL(pq16_decode_kernel, dim3((unsigned)nblocks), dim3(64 * KC), 0, s, d_codebooks, d_codes, d_off,
                       bo.p, nlist, M, dsub, KC, std::ldexp(1.0f, xexp), data.p);
    FDB_HIP(hipGetLastError());
    hipLaunchKernelGGL(pq16_norms_kernel, dim3((unsigned)cdiv(nblocks * 32, kT)), dim3(kT), 0, s, d_codebooks,
                       d_codes, d_off, bo.p, nlist, nblocks * 32, M, dsub, xnb.p, xmax2.p);
    FDB_HIP(hipGetLastError());
  }
  ok = true;
}

void Pq16Lists::build_rows(const float* d_rows, const uint32_t* d_off, const std::vector<uint64_t>& offsets,
                           uint32_t nl, int dim, hipStream_t s) {
  ok = false;
  M = 1;
  dsub = dim;
  D = dim;
  KC = (D + 15) / 16;
  nlist = nl;
  // the reference's squared L2 (8 FMA lanes, their sum, the tail): a term
  // is rounded at most dim + 2 times (its subtraction included)
  nref = dim + 2;
  if (KC > 16 || nlist == 0 || nlist > kHistMax || dim <= 0) return;
  std::vector<uint32_t> hbo(nlist + 1, 0);
  uint64_t nbk = 0;
  max_blocks = 0;
  for (uint32_t p = 0; p < nlist; ++p) {
    hbo[p] = (uint32_t)nbk;
    const uint64_t nb = cdiv(offsets[p + 1] - offsets[p], 32);
    nbk += nb;
    max_blocks = std::max(max_blocks, nb);
  }
  if (nbk >= 0xFFFFFFFFull || offsets[nlist] >= 0xFFFFFFFFull) return;
  hbo[nlist] = (uint32_t)nbk;
  nblocks = nbk;
  bo.upload(hbo.data(), hbo.size(), s);
  stats.reserve(1);
  hipLaunchKernelGGL(pq16_fill_u32, dim3(1), dim3(kT), 0, s, stats.p, (uint64_t)1, 0u);
  FDB_HIP(hipGetLastError());
  const uint64_t n = offsets[nlist] * (uint64_t)dim;
  if (n > 0) {
    hipLaunchKernelGGL(pq16_cb_stats_kernel, dim3((unsigned)std::min<uint64_t>(cdiv(n, kT), 1024)), dim3(kT), 0, s,
                       d_rows, n, stats.p);
    FDB_HIP(hipGetLastError());
  }
  uint32_t mbits = 0;
  FDB_HIP(hipMemcpyAsync(&mbits, stats.p, 4, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  if (mbits >= 0x7F800000u) return;  // a non-finite component
  float mxv;
  std::memcpy(&mxv, &mbits, 4);
  cmax = mxv;
  xexp = 0;
  if (mxv > 0.0f) {
    int E;
    (void)std::frexp(mxv, &E);
    xexp = 13 - E;
  }
  if (xexp > 100 || xexp < -100) return;
  data.reserve(std::max<uint64_t>(nblocks * KC * 64, 1));
  xnb.reserve(std::max<uint64_t>(nblocks * 32, 1));
  xmax2.reserve(nlist);
  hipLaunchKernelGGL(pq16_fill_u32, dim3((unsigned)std::min<uint64_t>(cdiv(nlist, kT), 1024)), dim3(kT), 0, s,
                     xmax2.p, (uint64_t)nlist, 0u);
  FDB_HIP(hipGetLastError());
  if (nblocks > 0) {
    hipLaunchKernelGGL(pq16_rows_kernel, dim3((unsigned)nblocks), dim3(64 * KC), 0, s, d_rows, d_off, bo.p, nlist, D,
                       KC, std::ldexp(1.0f, xexp), data.p);
    FDB_HIP(hipGetLastError());
    hipLaunchKernelGGL(pq16_row_norms_kernel, dim3((unsigned)cdiv(nblocks * 32, kT)), dim3(kT), 0, s, d_rows, d_off,
                       bo.p, nlist, nblocks * 32, D, xnb.p, xmax2.p);
    FDB_HIP(hipGetLastError());
  }
  ok = true;
}

void Pq16Searcher::reset_stats(hipStream_t) {
  stat_.reserve(4);
  clear_ = true;
  pending_nq_ = 0;
}

// The statistics of the last slice searched, from its flags and candidate
// counts (before the next slice overwrites them).
void Pq16Searcher::flush_stats(hipStream_t s) {
  if (pending_nq_ == 0) return;
  hipLaunchKernelGGL(pq16_stats_kernel, dim3(1), dim3(1024), 0, s, flags_.p, nreal_.p, pending_nq_, clear_ ? 1 : 0,
                     stat_.p);
  FDB_HIP(hipGetLastError());
  clear_ = false;
  pending_nq_ = 0;
}

Pq16Searcher::~Pq16Searcher() {
  for (auto& e : tev_)
    if (e) (void)hipEventDestroy(e);
}

void Pq16Searcher::set_timing(bool on) {
  timing_ = on;
  screen_ms_ = 0.0f;
  if (on)
    for (auto& e : tev_)
      if (!e) FDB_HIP(hipEventCreate(&e));
}

void Pq16Searcher::read_stats(uint64_t& fallbacks, uint64_t& candidates, hipStream_t s) {
  fallbacks = candidates = 0;
  flush_stats(s);
  if (!stat_.p || clear_) return;
  uint32_t v[4] = {0, 0, 0, 0};
  FDB_HIP(hipMemcpyAsync(v, stat_.p, 16, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  fallbacks = v[0];
  candidates = (uint64_t)v[2] | ((uint64_t)v[3] << 32);
}

void Pq16Searcher::search(const Pq16Lists& L, const Pq16SearchArgs& a, hipStream_t s) {
  const uint64_t nq = a.nq;
  if (nq == 0) return;
  const uint32_t nlist = L.nlist;
  const int np = a.np;
  if (np < 1) throw Error(FDB_ERR_INVALID_ARGUMENT, "screened search: nprobe < 1");
  const uint32_t cap = capacity(a.k);
  const uint64_t npr = nq * (uint64_t)np;
  if (ncu_ == 0) {
    int dev = 0, v = 0;
    FDB_HIP(hipGetDevice(&dev));
    FDB_HIP(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev));
    ncu_ = std::max(v, 1);
  }
  if (cnt_.n < 2ull * nlist) {  // the list counts start zero; every search leaves them zero
    cnt_.reserve(2ull * nlist);
    cnt_clean_ = false;
  }
  if (!cnt_clean_) {
    hipLaunchKernelGGL(pq16_fill_u32, dim3((unsigned)cdiv(2ull * nlist, kT)), dim3(kT), 0, s, cnt_.p,
                       2ull * nlist, 0u);
    FDB_HIP(hipGetLastError());
    cnt_clean_ = true;
  }
  qoff_.reserve(2 * (uint64_t)(nlist + 1));
  toff_.reserve(2 * (uint64_t)(nlist + 1));
  tcnt_.reserve(2ull * nlist);
  tctr_.reserve(2 * kXcd);
  qlist_.reserve(2 * std::max<uint64_t>(npr, 1));
  jlim_.reserve(nq);
  offA_.reserve(npr);
  nA_.reserve(nq);
  nreal_.reserve(nq);
  epsA_.reserve(npr);
  const uint32_t capA = cap_first(a.k);
  bufA_.reserve(nq * capA);
  dkA_.reserve(nq);
  ccnt_.reserve(nq);
  cand_.reserve(nq * cap);
  force_.reserve(nq);
  flags_.reserve(nq);
  if (!stat_.p) reset_stats(s);
  flush_stats(s);  // the previous slice's, before its buffers are reused
  nheavy_.reserve(4);
  order_.reserve(nq);
  hipLaunchKernelGGL(pq16_plan_kernel, dim3((unsigned)cdiv(nq, kT)), dim3(kT), 0, s, a.probes, nq, np, nlist,
                     a.list_off, a.k, capA, jlim_.p, offA_.p, nA_.p, nreal_.p, ccnt_.p, force_.p, epsA_.p,
                     nheavy_.p);
  FDB_HIP(hipGetLastError());

  // (query, probe) pairs grouped by list, stage st (0: first lists, 1: all)
  const uint32_t G =
      (uint32_t)std::min<uint64_t>(std::max<uint64_t>(cdiv(npr, (uint64_t)kSortT * kSortB), 1), kSortWG);
  const uint64_t chunk = cdiv(npr, G);
  // tiles of a stage: at most (pairs / 128 + lists) pair tiles per chunk
  // Large indexes (tens of tiles per resident workgroup) take their tiles
  // from per-XCD counters in descending order of size, so that the last
  // tiles are short.  Measured at 10M x 96 codes (nlist 4096, nprobe 64):
  // stage B 1.56-1.60 ms against 1.81 with the static stride; at 1M x 128
  // (nlist 1024, nprobe 16; ~3 tiles per workgroup) the static stride over
  // tiles in list order was faster (0.175 against 0.185 ms).  Sorted tiles
  // hold up to kCBDyn blocks: fewer tiles, so less of the per-tile setup.
  const bool dyn = a.tiles >= 0 ? a.tiles == 1 : L.nblocks >= 512ull * (uint64_t)ncu_;
  const uint32_t cbB = dyn ? kCBDyn : kCB;
  const uint32_t cbA = dyn ? kCBDyn : kCB;
  auto tile_bound = [&](uint32_t blim, uint32_t cb) {
    return (cdiv(npr, kTilePairs) + nlist) * cdiv(std::min<uint64_t>(L.max_blocks, blim), cb);
  };
  const uint64_t tbA = tile_bound(capA / 32, cbA), tbB = tile_bound(0xFFFFFFFFu, cbB);
  desc_.reserve(std::max<uint64_t>(tbA + tbB, 1));
  // both stages' pairs grouped by list: 0 the first lists, 1 every probe
  PairStages pst{};
  pst.s0 = PairSet{a.probes, nq, np, jlim_.p, nlist, chunk};
  pst.s1 = PairSet{a.probes, nq, np, nullptr, nlist, chunk};
  pst.blim0 = capA / 32;
  pst.blim1 = 0xFFFFFFFFu;
  pst.tq0 = kTilePairs;
  const int wvB = stage_b_wgwaves(L.KC);
  pst.sort = dyn ? 1u : 0u;
  pst.tq1 = 32 * wvB * stage_b_groups(L.KC);
  pst.cb0 = cbA;
  pst.cb1 = cbB;
  pst.cnt = cnt_.p;
  pst.qoff = qoff_.p;
  pst.toff = toff_.p;
  pst.tcnt = tcnt_.p;
  pst.tctr = tctr_.p;
  pst.qlist = qlist_.p;
  pst.desc = desc_.p;
  pst.npr = std::max<uint64_t>(npr, 1);
  pst.tl1 = tbA;
  cnt_clean_ = false;  // until the scatter has run
  hipLaunchKernelGGL(pq16_count_kernel, dim3(G, 2), dim3(kSortT), 0, s, pst);
  FDB_HIP(hipGetLastError());
  hipLaunchKernelGGL(pq16_offsets_kernel, dim3(2), dim3(kSortT), 0, s, pst, L.bo.p);
  FDB_HIP(hipGetLastError());
  hipLaunchKernelGGL(pq16_scatter_kernel, dim3(G, 2), dim3(kSortT), 0, s, pst, L.bo.p);
  FDB_HIP(hipGetLastError());
  cnt_clean_ = true;

  ScreenArgs sa{};
  sa.queries = a.queries;
  sa.D = L.D;
  sa.vec = L.D == 16 * L.KC && (reinterpret_cast<uintptr_t>(a.queries) & 15) == 0 &&
           (a.rows || (reinterpret_cast<uintptr_t>(a.centroids) & 15) == 0);
  sa.centroids = a.rows ? nullptr : a.centroids;  // full vectors: the query is the residual
  sa.list_off = a.list_off;
  sa.bo = L.bo.p;
  sa.data = L.data.p;
  sa.xnb = L.xnb.p;
  sa.xmax2 = L.xmax2.p;
  sa.nlist = nlist;
  sa.np = np;
  sa.xexp = L.xexp;
  sa.bufA = bufA_.p;
  sa.offA = offA_.p;
  sa.epsA = epsA_.p;
  sa.capA = capA;
  sa.dkA = dkA_.p;
  sa.ccnt = ccnt_.p;
  sa.cand = cand_.p;
  sa.cap = cap;
  sa.force = force_.p;
  pq16_eps_coeffs(16 * L.KC, L.nref, L.cmax, sa.c_dot, sa.c_sq, sa.cabs);
  void (*dense)(ScreenArgs) = nullptr;
  void (*thresh)(ScreenArgs) = nullptr;
  switch (L.KC) {
#define FDB_KC(n)                                  \
  case n:                                          \
    dense = pq16_dense_kernel<n>;                  \
    thresh = thresh_kernel<n>();                   \
    break;
    FDB_KC(1) FDB_KC(2) FDB_KC(3) FDB_KC(4) FDB_KC(5) FDB_KC(6) FDB_KC(7) FDB_KC(8)
    FDB_KC(9) FDB_KC(10) FDB_KC(11) FDB_KC(12) FDB_KC(13) FDB_KC(14) FDB_KC(15) FDB_KC(16)
#undef FDB_KC
  }
  if (!dense) throw Error(FDB_ERR_HIP, "no screening kernel for this dimension");
  // Dynamic tiles: one resident round of workgroups (a multiple of kXcd),
  // which then take tiles from their XCD's counter.  Static: eight
  // workgroups per CU striding over the tiles (a multiple of kXcd * run).
  auto grid_of = [&](void (*kern)(ScreenArgs), int threads) {
    if (!dyn) return (unsigned)(std::max<uint64_t>(cdiv(8 * (uint64_t)ncu_, kXcd * kXcdRun), 1) * kXcd * kXcdRun);
    for (const auto& g : grids_)
      if (g.first == reinterpret_cast<const void*>(kern)) return g.second;
    int per = 0;
    FDB_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kern, threads, 0));
    const unsigned g = (unsigned)(std::max<uint64_t>(cdiv((uint64_t)std::max(per, 1) * ncu_, kXcd), 1) * kXcd);
    grids_.emplace_back(reinterpret_cast<const void*>(kern), g);
    return g;
  };

  // 1. the first lists of each query, every screened value kept; d_k bound
  sa.qoff = qoff_.p;
  sa.toff = toff_.p;
  sa.desc = desc_.p;
  sa.qlist = qlist_.p;
  sa.blim = capA / 32;
  sa.cb = cbA;
  sa.tctr = tctr_.p;
  sa.dyn = dyn ? 1u : 0u;
  sa.run = dyn ? kXcdRunDyn : kXcdRun;
  hipLaunchKernelGGL(dense, dim3(grid_of(dense, 256)), dim3(256), 0, s, sa);
  FDB_HIP(hipGetLastError());
  const int R = list_regs(a.k);
  switch (R) {
#define FDB_SEL(n)                                                                                              \
  case n:                                                                                                       \
    hipLaunchKernelGGL(pq16_select_kernel<n>, dim3((unsigned)nq), dim3(64), 0, s, bufA_.p, capA, nA_.p, nreal_.p, jlim_.p, \
                       epsA_.p, np, a.k, a.rows && a.sqrt_out ? 1 : 0, dkA_.p);                                 \
    break;
    FDB_SEL(1) FDB_SEL(2) FDB_SEL(4) FDB_SEL(8) FDB_SEL(16)
#undef FDB_SEL
    default:
      throw Error(FDB_ERR_UNSUPPORTED, "k above 1024");
  }
  FDB_HIP(hipGetLastError());

  // 2. every probed list against the bound
  sa.qoff = qoff_.p + (nlist + 1);
  sa.toff = toff_.p + (nlist + 1);
  sa.desc = desc_.p + tbA;
  sa.qlist = qlist_.p + std::max<uint64_t>(npr, 1);
  sa.blim = 0xFFFFFFFFu;
  sa.cb = cbB;
  sa.tctr = tctr_.p + kXcd;
  const unsigned gridB = grid_of(thresh, 64 * wvB);
  if (timing_) FDB_HIP(hipEventRecord(tev_[0], s));
  hipLaunchKernelGGL(thresh, dim3(gridB), dim3(64 * wvB), 0, s, sa);
  FDB_HIP(hipGetLastError());
  if (timing_) {
    FDB_HIP(hipEventRecord(tev_[1], s));
    FDB_HIP(hipEventSynchronize(tev_[1]));
    float ms = 0.0f;
    FDB_HIP(hipEventElapsedTime(&ms, tev_[0], tev_[1]));
    screen_ms_ += ms;
  }

  // 3. exact distances of the candidates
  RescoreArgs16 r{};
  r.queries = a.queries;
  r.D = L.D;
  r.M = L.M;
  r.dsub = L.dsub;
  r.probes = a.probes;
  r.np = np;
  r.centroids = a.centroids;
  r.codebooks = a.codebooks;
  r.codes = a.codes;
  r.ids = a.ids;
  r.ccnt = ccnt_.p;
  r.cand = cand_.p;
  r.cap = cap;
  r.force = force_.p;
  r.k = a.k;
  r.order = a.order;
  r.rows = a.rows;
  r.sqrt_out = a.sqrt_out;
  r.out_ids = a.out_ids;
  r.out_d = a.out_d;
  r.out_counts = a.out_counts;
  r.flags = flags_.p;
  r.nexp = nreal_.p;  // free after the d_k selection
  // part slots: every heavy part of the slice, within 256 MiB of lists
  const uint64_t pmax = std::max<uint64_t>(
      1, std::min<uint64_t>(nq * cdiv(cap, kPart), (256ull << 20) / (8ull * (uint64_t)a.k)));
  heavy_.reserve(pmax);
  multi_.reserve(nq);
  part_d_.reserve(pmax * a.k);
  part_k_.reserve(pmax * a.k);
  r.heavy = heavy_.p;
  r.pmax = (uint32_t)pmax;
  r.part_d = part_d_.p;
  r.part_k = part_k_.p;
  r.qorder = order_.p;
  r.counters = nheavy_.p;
  r.cb4 = L.cb4.p;
  r.nlist = (int)nlist;
  r.cached = !a.rows && (uint64_t)np * L.D * sizeof(float) <= 32 * 1024;
  const size_t lds = sizeof(float) * ((size_t)L.D + (r.cached ? (size_t)np * L.D : 0));
  const int ds = (L.dsub == 3 || L.dsub == 4 || L.dsub == 8) ? L.dsub : 0;
  void (*rk)(RescoreArgs16, uint64_t, uint32_t) = nullptr;
#define FDB_RS(n)                                                                       \
  case n:                                                                               \
    rk = a.rows ? pq16_rescore_kernel<n, -1, 0>                                                      \
         : ds == 3 ? (L.M == 32 ? pq16_rescore_kernel<n, 3, 32> : pq16_rescore_kernel<n, 3, 0>)      \
                 : (ds == 4 ? pq16_rescore_kernel<n, 4, 0>                                           \
                            : (ds == 8 ? (L.M == 16 ? pq16_rescore_kernel<n, 8, 16> : pq16_rescore_kernel<n, 8, 0>) \
                                       : pq16_rescore_kernel<n, 0, 0>));                             \
    break;
  switch (R) { FDB_RS(1) FDB_RS(2) FDB_RS(4) FDB_RS(8) FDB_RS(16) }
#undef FDB_RS
  hipLaunchKernelGGL(pq16_classify_kernel, dim3((unsigned)cdiv(nq, kT)), dim3(kT), 0, s, ccnt_.p, force_.p, cap, nq,
                     flags_.p, order_.p, heavy_.p, (uint32_t)pmax, multi_.p, nreal_.p, nheavy_.p);
  FDB_HIP(hipGetLastError());
  const uint32_t nh = (uint32_t)std::min<uint64_t>(nq, 2 * (uint64_t)ncu_);  // heavy-list workgroups
  hipLaunchKernelGGL(rk, dim3((unsigned)(nh + cdiv(nq, kT / 64))), dim3(kT), lds, s, r, nq, nh);
  FDB_HIP(hipGetLastError());
  const unsigned mg = (unsigned)std::min<uint64_t>(nq, 4 * (uint64_t)ncu_);
  switch (R) {
#define FDB_MG(n)                                                                  \
  case n:                                                                          \
    hipLaunchKernelGGL((pq16_merge_kernel<n, merge_waves(n)>), dim3(mg), dim3(64 * merge_waves(n)), 0, s, r, multi_.p); \
    break;
    FDB_MG(1) FDB_MG(2) FDB_MG(4) FDB_MG(8) FDB_MG(16)
#undef FDB_MG
  }
  FDB_HIP(hipGetLastError());
  pending_nq_ = nq;  // counted by flush_stats
}

}  // namespace fdb
