// Coarse selection screened on the matrix cores; the method and its bound
// are described in fdb_coarse16.hpp.
//
// c16_stats_kernel     largest |component| of the centroids (non-finite
//                      values compare above every finite one)
// c16_blocks_kernel    fp16 A-operand blocks of 32 centroids and their
//                      norms, laid out per half-lane
// coarse16_kernel      4 waves per 32 queries: the bound pass and the
//                      candidate pass; each query's candidates to a list
// coarse16_rescore_kernel
//                      a wave per query: exact rescoring of its candidates
//                      and selection (many more workgroups than tiles)
#include "fdb_coarse16.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

#include "fdb_device.hpp"

namespace fdb {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kT = 256;
constexpr int kW = 4;              // waves per coarse16_kernel workgroup
constexpr int kCT = 64 * kW;
constexpr int kBadExp = 1 << 20;  // scale exponent of a query not screened
constexpr int kMaxCap = 128;       // candidate slots per query at nprobe 64

uint64_t cdiv(uint64_t a, uint64_t b) { return (a + b - 1) / b; }

__global__ __launch_bounds__(kT) void c16_stats_kernel(const float* __restrict__ c, uint64_t n,
                                                       uint32_t* __restrict__ stats) {
  uint32_t m = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * kT + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kT)
    m = max(m, __float_as_uint(c[i]) & 0x7FFFFFFFu);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (uint32_t)__shfl_xor((int)m, off));
  if ((threadIdx.x & 63) == 0) atomicMax(&stats[0], m);
}

// Workgroup (64 * KC threads) per block of 32 centroids: thread (kc, lane)
// writes the 8 halves of centroid 32b + lane%32 on dimensions 16kc +
// 8(lane/32) .. +7 (zero past nlist and dim), scaled by 2^xexp.  Threads of
// k-chunk 0 also write |c|^2 (fp32, dimension order; +inf past nlist) to
// cnp[b][h][i] for the half-lane h = (row / 4) % 2 that holds row
// 8(i/4) + 4h + i%4 in the MFMA output, and the largest |c|^2 to stats[1].
__global__ void c16_blocks_kernel(const float* __restrict__ cen, uint32_t nlist, int dim, int KC, float scale,
                                  uint4* __restrict__ out, float* __restrict__ cnp, uint32_t* __restrict__ stats) {
  const uint32_t b = blockIdx.x;
  const int kc = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const uint32_t c = b * 32 + (lane & 31);
  const bool valid = c < nlist;
  _Float16 h[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int d = kc * 16 + 8 * (lane >> 5) + t;
    h[t] = (_Float16)(valid && d < dim ? cen[(uint64_t)c * dim + d] * scale : 0.0f);
  }
  uint4 w;
  w.x = (uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16);
  w.y = (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16);
  w.z = (uint32_t)__builtin_bit_cast(uint16_t, h[4]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[5]) << 16);
  w.w = (uint32_t)__builtin_bit_cast(uint16_t, h[6]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[7]) << 16);
  out[((uint64_t)b * KC + kc) * 64 + lane] = w;
  if (kc == 0 && lane < 32) {
    float s = f_inf();
    if (valid) {
      s = 0.0f;
      for (int d = 0; d < dim; ++d) {
        const float v = cen[(uint64_t)c * dim + d];
        s = __builtin_fmaf(v, v, s);
      }
      atomicMax(&stats[1], __float_as_uint(s));
    }
    const int row = lane;
    const int hh = (row >> 2) & 1;
    const int i = 4 * (row >> 3) + (row & 3);
    cnp[(uint64_t)b * 32 + hh * 16 + i] = s;
  }
}

// a + b rounded up past the exact sum (either sign; no overflow): the
// rounded sum is within 2^-24 |t| of it, and 2^-22 |t| added to t rounds to
// at least t + 2^-23 |t|
__device__ __forceinline__ float add_up(float a, float b) {
  const float t = a + b;
  return t + __builtin_fabsf(t) * 0x1p-22f;
}

struct C16Args {
  const float* queries;
  uint64_t nq;
  int dim;
  int vec;  // centroid rows start 16-byte aligned (dim % 4 == 0)
  const float* centroids;
  uint32_t nlist, nblk;
  const uint4* blocks;
  const float* cnp;
  int xexp;
  float c_dot, c_sq, cabs, xnorm;
  int np, cap;
  int32_t* probes;
  float* dists;
  int* flags;
  uint32_t* cand;  // [nq][cap] screened candidates (centroid indices)
  uint32_t* ncand; // [nq] their count (0 for a flagged query)
};

// Sorted insertion of v into the m smallest kept in t[0..M) ascending.
template <int M>
__device__ __forceinline__ void keep_smallest(float (&t)[M], float v) {
#pragma unroll
  for (int i = M - 1; i > 0; --i) t[i] = fminf(t[i], fmaxf(t[i - 1], v));
  t[0] = fminf(t[0], v);
}

// Sorts a bitonic sequence ascending (N a power of two).
template <int N>
__device__ __forceinline__ void bitonic_clean(float (&a)[N]) {
#pragma unroll
  for (int k = N / 2; k >= 1; k >>= 1)
#pragma unroll
    for (int i = 0; i < N; ++i)
      if ((i & k) == 0) {
        const float lo = fminf(a[i], a[i + k]);
        const float hi = fmaxf(a[i], a[i + k]);
        a[i] = lo;
        a[i + k] = hi;
      }
}

// c = the 2L values of ascending a and b, ascending (a then b reversed is
// bitonic)
template <int L>
__device__ __forceinline__ void merge_all(const float (&a)[L], const float (&b)[L], float (&c)[2 * L]) {
#pragma unroll
  for (int i = 0; i < L; ++i) {
    c[i] = a[i];
    c[L + i] = b[L - 1 - i];
  }
  bitonic_clean<2 * L>(c);
}

// c = the L smallest values of ascending a and b, ascending
template <int L>
__device__ __forceinline__ void merge_low(const float (&a)[L], const float (&b)[L], float (&c)[L]) {
#pragma unroll
  for (int i = 0; i < L; ++i) c[i] = fminf(a[i], b[L - 1 - i]);
  bitonic_clean<L>(c);
}

// Workgroup of kW waves per tile of 32 queries.  Lane l of a wave serves
// query l % 32 with the half-lane l / 32; wave w screens the blocks w, w +
// kW, ...  M: block minima kept per (wave, half-lane), 2 kW M >= np.
// LDS: the tile's queries (fp32, rows of 16 KC, stride 16 KC + 4), then
// per query cap candidate slots (centroid index, distance bits); before the
// candidate pass the slots hold the kept minima, [32][2 kW M + 4].
template <int KC, int M>
__global__ __launch_bounds__(kCT) __attribute__((amdgpu_waves_per_eu(2))) void coarse16_kernel(C16Args a) {
  constexpr int LDQ = 16 * KC;      // floats of a query row
  constexpr int LQS = LDQ + 4;      // their LDS stride: 4 banks apart (no conflicts across rows)
  constexpr int U = 2 * kW * M;  // kept minima per query
  constexpr int US = U + 4;      // their LDS stride (4 banks apart)
  static_assert(U % 64 == 0, "kept minima fill whole waves");
  extern __shared__ __align__(16) uint32_t lds[];
  __shared__ float s_qn[32], s_T[32];
  __shared__ int s_eq[32];
  __shared__ uint32_t s_cnt[32], s_pre[33];
  __shared__ uint8_t s_pair[M == 16 ? 1 : 32 * kMaxCap];  // query of each rescored pair (in-kernel rescoring)
  float* __restrict__ qs = reinterpret_cast<float*>(lds);
  uint2* __restrict__ cand = reinterpret_cast<uint2*>(lds + 32 * LQS);
  float* __restrict__ mins = reinterpret_cast<float*>(cand);
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 31;
  const int half = lane >> 5;
  const uint64_t q0 = (uint64_t)blockIdx.x * 32;
  const int nqt = (int)min<uint64_t>(32, a.nq - q0);
  const int cap = a.cap;

  // the tile's queries, zero past dim and past the last query (every load
  // issued before the first store)
  {
    constexpr int R = 32 * LDQ / kCT;
    static_assert(32 * LDQ % kCT == 0, "whole rows of the tile per pass");
    float v[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = tid + r * kCT;
      const int qi = e / LDQ;
      const int d = e - qi * LDQ;
      v[r] = (qi < nqt && d < a.dim) ? a.queries[(q0 + qi) * (uint64_t)a.dim + d] : 0.0f;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int e = tid + r * kCT;
      const int qi = e / LDQ;
      qs[qi * LQS + (e - qi * LDQ)] = v[r];
    }
  }
  if (tid < 32) s_cnt[tid] = 0;
  __syncthreads();
  // per query: |q|^2 in fp32 and the scale exponent (TPQ threads a query)
  {
    constexpr int TPQ = kCT / 32;
    static_assert((TPQ & (TPQ - 1)) == 0 && TPQ <= 64, "threads per query: a power of two within a wave");
    const int qi = tid / TPQ, sub = tid % TPQ;
    float mx = 0.0f, qn = 0.0f;
    int nan = 0;
#pragma unroll
    for (int i = 0; i < LDQ / TPQ; ++i) {
      const float v = qs[qi * LQS + sub + i * TPQ];
      nan |= v != v;
      mx = fmaxf(mx, __builtin_fabsf(v));
      qn = __builtin_fmaf(v, v, qn);
    }
#pragma unroll
    for (int off = TPQ / 2; off > 0; off >>= 1) {
      mx = fmaxf(mx, __shfl_xor(mx, off));
      qn = qn + __shfl_xor(qn, off);
      nan |= __shfl_xor(nan, off);
    }
    if (sub == 0) {
      int eq = 0;
      if (mx > 0.0f) {
        int E;
        (void)frexpf(mx, &E);
        eq = 13 - E;  // mx * 2^eq in [2^12, 2^13)
      }
      const bool bad = nan || !(qn <= 3.0e38f) || eq > 100 || eq < -100 || qi >= nqt;
      s_qn[qi] = qn;
      s_eq[qi] = bad ? kBadExp : eq;
    }
  }
  __syncthreads();

  // the lane's B operand: its query scaled by 2^eq, halves on dimensions
  // 16kc + 8(l/32) .. +7
  const int eqv = s_eq[col];
  const int eq = eqv == kBadExp ? 0 : eqv;
  const float sc = ldexpf(1.0f, eq);
  v8h bq[KC];
#pragma unroll
  for (int kc = 0; kc < KC; ++kc) {
    const float4 x0 = *reinterpret_cast<const float4*>(qs + col * LQS + kc * 16 + 8 * half);
    const float4 x1 = *reinterpret_cast<const float4*>(qs + col * LQS + kc * 16 + 8 * half + 4);
    bq[kc][0] = (_Float16)(x0.x * sc);
    bq[kc][1] = (_Float16)(x0.y * sc);
    bq[kc][2] = (_Float16)(x0.z * sc);
    bq[kc][3] = (_Float16)(x0.w * sc);
    bq[kc][4] = (_Float16)(x1.x * sc);
    bq[kc][5] = (_Float16)(x1.y * sc);
    bq[kc][6] = (_Float16)(x1.z * sc);
    bq[kc][7] = (_Float16)(x1.w * sc);
  }
  const float cneg = -ldexpf(1.0f, 1 - eq - a.xexp);
  const v4u* __restrict__ A = reinterpret_cast<const v4u*>(a.blocks);

  // Block operands (A chunks and the lane's 16 norms), loaded one block
  // ahead of their use.
  struct Ops {
    v4u av[KC];
    float4 xn[4];
  };
  auto load = [&](uint32_t b, Ops& o) {
    const v4u* __restrict__ ab = A + (uint64_t)b * KC * 64 + lane;
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) o.av[kc] = ab[kc * 64];
    const float4* __restrict__ xn = reinterpret_cast<const float4*>(a.cnp + (uint64_t)b * 32 + half * 16);
#pragma unroll
    for (int g = 0; g < 4; ++g) o.xn[g] = xn[g];
  };
  // the 16 screened values of the lane's rows of a block: |c|^2 - 2<q, c>
  // (the query's |q|^2 is the same for all its centroids and is left out)
  auto screen = [&](const Ops& o, float* s) {
    v16f acc = {};
#pragma unroll
    for (int kc = 0; kc < KC; ++kc)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, o.av[kc]), bq[kc], acc, 0, 0, 0);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      s[4 * g] = __builtin_fmaf(cneg, acc[4 * g], o.xn[g].x);
      s[4 * g + 1] = __builtin_fmaf(cneg, acc[4 * g + 1], o.xn[g].y);
      s[4 * g + 2] = __builtin_fmaf(cneg, acc[4 * g + 2], o.xn[g].z);
      s[4 * g + 3] = __builtin_fmaf(cneg, acc[4 * g + 3], o.xn[g].w);
    }
  };
  // the wave's blocks once, in order, their operands fetched two ahead
  // (three register sets taken in turn), or one ahead past 128 dimensions.
  // Fetches past the wave's last block read the table's last block instead
  // (unused): unconditional loads keep the count of loads in flight the same
  // on every path, so each wait is for the one set about to be used.
  auto sweep = [&](auto&& f) {
    const uint32_t n = a.nblk, st = kW;
    uint32_t b = (uint32_t)wave;
    if (b >= n) return;
    auto at = [&](uint32_t x) { return x < n ? x : n - 1; };
    float s[16];
    if constexpr (KC > 8) {
      Ops cur, nxt;
      load(b, cur);
      for (;; b += st) {
        load(at(b + st), nxt);
        screen(cur, s);
        f(b, s);
        if (b + st >= n) break;
        cur = nxt;
      }
      return;
    }
    Ops o0, o1, o2;
    load(b, o0);
    load(at(b + st), o1);
    for (;; b += 3 * st) {
      load(at(b + 2 * st), o2);
      screen(o0, s);
      f(b, s);
      if (b + st >= n) break;
      load(at(b + 3 * st), o0);
      screen(o1, s);
      f(b + st, s);
      if (b + 2 * st >= n) break;
      load(at(b + 4 * st), o1);
      screen(o2, s);
      f(b + 2 * st, s);
      if (b + 3 * st >= n) break;
    }
  };

  // pass 1: the M smallest block minima of the lane's half of its blocks
  float top[M];
#pragma unroll
  for (int i = 0; i < M; ++i) top[i] = f_inf();
  sweep([&](uint32_t, const float* s) {
    const float m = fminf(fminf(fminf(fminf(s[0], s[1]), fminf(s[2], s[3])), fminf(fminf(s[4], s[5]), fminf(s[6], s[7]))),
                          fminf(fminf(fminf(s[8], s[9]), fminf(s[10], s[11])),
                                fminf(fminf(s[12], s[13]), fminf(s[14], s[15]))));
    if (__ballot(m < top[M - 1]) != 0) keep_smallest<M>(top, m);
  });
#pragma unroll
  for (int i = 0; i < M; ++i) mins[col * US + (wave * 2 + half) * M + i] = top[i];
  __syncthreads();

  // S = the np-th smallest kept minimum (they belong to distinct
  // centroids), T = S + 2 eps rounded up; -inf where the query is not
  // screened.  Wave 0, lane q + 32h: query q's lists 4h .. 4h+3 (each
  // ascending), merged in registers; the two halves' 4M smallest are
  // exchanged and merged once more (np <= 4M).
  static_assert(kW == 4, "eight kept lists per query: four per half-wave");
  if (wave == 0) {
    const float* __restrict__ mq = mins + col * US + 4 * half * M;
    float l0[M], l1[M], l2[M], l3[M];
#pragma unroll
    for (int i = 0; i < M; i += 4) {
      const float4 x0 = *reinterpret_cast<const float4*>(mq + i);
      const float4 x1 = *reinterpret_cast<const float4*>(mq + M + i);
      const float4 x2 = *reinterpret_cast<const float4*>(mq + 2 * M + i);
      const float4 x3 = *reinterpret_cast<const float4*>(mq + 3 * M + i);
      l0[i] = x0.x, l0[i + 1] = x0.y, l0[i + 2] = x0.z, l0[i + 3] = x0.w;
      l1[i] = x1.x, l1[i + 1] = x1.y, l1[i + 2] = x1.z, l1[i + 3] = x1.w;
      l2[i] = x2.x, l2[i + 1] = x2.y, l2[i + 2] = x2.z, l2[i + 3] = x2.w;
      l3[i] = x3.x, l3[i + 1] = x3.y, l3[i + 2] = x3.z, l3[i + 3] = x3.w;
    }
    float a01[2 * M], a23[2 * M], f[4 * M], g[4 * M], lo[4 * M];
    merge_all<M>(l0, l1, a01);
    merge_all<M>(l2, l3, a23);
    merge_all<2 * M>(a01, a23, f);
#pragma unroll
    for (int i = 0; i < 4 * M; ++i) g[i] = __shfl_xor(f[i], 32);
    merge_low<4 * M>(f, g, lo);
    // lo ascending: the np-th smallest, with no indexed register access
    float S = lo[0];
#pragma unroll
    for (int i = 1; i < 4 * M; ++i) S = i < a.np ? lo[i] : S;
    if (half == 0) {
      const float qnq = s_qn[col];
      const float qnorm = sqrtf(qnq) * (1.0f + 0x1p-16f);
      const float Xp = a.xnorm + a.cabs;
      const float tt = qnorm + Xp;
      const float eps = a.c_dot * qnorm * Xp + a.c_sq * tt * tt + 1e-30f;
      const bool act = s_eq[col] != kBadExp && S < f_inf();
      s_T[col] = act ? add_up(S, add_up(eps, eps)) : -f_inf();
    }
  }
  __syncthreads();

  // pass 2: every centroid with s <= T to the query's slots
  const float T = s_T[col];
  sweep([&](uint32_t b, const float* s) {
    // rows past nlist never pass (a threshold of +inf would let them)
    const uint32_t cb = b * 32 + 4 * half;
    uint32_t passm = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r)
      passm |= (s[r] <= T && cb + 8 * (r >> 2) + (r & 3) < a.nlist ? 1u : 0u) << r;
    if (__ballot(passm != 0) == 0) return;
    if (passm == 0) return;
    uint32_t pos = atomicAdd(&s_cnt[col], (uint32_t)__popc(passm));
    while (passm) {
      const int r = __ffs(passm) - 1;
      passm &= passm - 1;
      if (pos < (uint32_t)cap) cand[col * cap + pos] = make_uint2(cb + 8 * (r >> 2) + (r & 3), 0u);
      ++pos;
    }
  });
  __syncthreads();

  if constexpr (M == 16) {
    // np > 32: the candidates go to coarse16_rescore_kernel (many more
    // workgroups than tiles for the larger rescoring and selection)
    // a query is served when it was screened and its candidates fit; the
    // others are flagged for the exact kernel.  The served queries' candidate
    // lists go to the rescoring kernel.
    {
      constexpr int TPQ = kCT / 32;
      const int qi = tid / TPQ, sub = tid % TPQ;
      const uint32_t n = s_cnt[qi];
      const bool ok = qi < nqt && s_T[qi] != -f_inf() && n >= (uint32_t)a.np && n <= (uint32_t)cap;
      if (qi < nqt) {
        if (sub == 0) {
          a.flags[q0 + qi] = ok ? 0 : 1;
          a.ncand[q0 + qi] = ok ? n : 0u;
        }
        if (ok)
          for (uint32_t j = (uint32_t)sub; j < n; j += TPQ) a.cand[(q0 + qi) * (uint64_t)cap + j] = cand[qi * cap + j].x;
      }
    }
    return;
  } else {
    // a query is served here when it was screened and its candidates fit;
    // the others are flagged for the exact kernel
    if (tid < 32) {
      const uint32_t n = s_cnt[tid];
      const bool ok = tid < nqt && s_T[tid] != -f_inf() && n >= (uint32_t)a.np && n <= (uint32_t)cap;
      if (tid < nqt) a.flags[q0 + tid] = ok ? 0 : 1;
      const uint32_t own = ok ? n : 0u;
      uint32_t inc = own;
#pragma unroll
      for (int off = 1; off < 32; off <<= 1) {
        const uint32_t v = (uint32_t)__shfl_up((int)inc, off);
        if (lane >= off) inc += v;
      }
      s_pre[tid + 1] = inc;
      if (tid == 0) s_pre[0] = 0;
      if (!ok) s_cnt[tid] = 0;
      // slots up to the next multiple of 16 hold a key above every candidate
      // (distance bits 0xFFFFFFFF are a NaN, which no distance is)
      if (ok)
        for (uint32_t j = n; j < (n + 15) / 16 * 16; ++j) cand[tid * cap + j] = make_uint2(0xFFFFFFFFu, 0xFFFFFFFFu);
    }
    __syncthreads();
    {
      constexpr int TPQ = kCT / 32;
      const int qi = tid / TPQ;
      const uint32_t b0 = s_pre[qi], n = s_pre[qi + 1] - b0;
      for (uint32_t j = (uint32_t)(tid % TPQ); j < n; j += TPQ) s_pair[b0 + j] = (uint8_t)qi;
    }
    __syncthreads();

    // rescoring: the exact distance of every (query, candidate) pair in the
    // reference's order, two threads a pair: thread h holds the FMA lanes
    // 4h .. 4h+3 over the 8-float chunks; lanes summed 0..7 in order, then
    // the scalar tail
    const uint32_t total = __builtin_amdgcn_readfirstlane(s_pre[32]);
    const int d8 = a.dim / 8;
    const int h = tid & 1;
    for (uint32_t i = (uint32_t)(tid >> 1); i < total; i += kCT / 2) {
      const int qi = s_pair[i];
      const uint32_t slot = i - s_pre[qi];
      const float* __restrict__ cr = a.centroids + (uint64_t)cand[qi * cap + slot].x * a.dim;
      const float* __restrict__ qr = qs + qi * LQS;
      float l0 = 0.0f, l1 = 0.0f, l2 = 0.0f, l3 = 0.0f;
      // the row's chunks loaded 16 at a time (d8 <= 2 KC), then the lanes
      constexpr int G = 2 * KC < 16 ? 2 * KC : 16;
#pragma unroll
      for (int j0 = 0; j0 < 2 * KC; j0 += G) {
        v4f x[G];
#pragma unroll
        for (int j = 0; j < G; ++j)
          if (j0 + j < d8) {
            const float* __restrict__ c8 = cr + 8 * (j0 + j) + 4 * h;
            if (a.vec) {
              x[j] = *reinterpret_cast<const v4f*>(c8);
            } else {
              x[j].x = c8[0];
              x[j].y = c8[1];
              x[j].z = c8[2];
              x[j].w = c8[3];
            }
          }
#pragma unroll
        for (int j = 0; j < G; ++j)
          if (j0 + j < d8) {
            const v4f y = *reinterpret_cast<const v4f*>(qr + 8 * (j0 + j) + 4 * h);
            const float e0 = y.x - x[j].x, e1 = y.y - x[j].y, e2 = y.z - x[j].z, e3 = y.w - x[j].w;
            l0 = __builtin_fmaf(e0, e0, l0);
            l1 = __builtin_fmaf(e1, e1, l1);
            l2 = __builtin_fmaf(e2, e2, l2);
            l3 = __builtin_fmaf(e3, e3, l3);
          }
      }
      const float lo = ((l0 + l1) + l2) + l3;
      const float from_lo = __shfl(lo, lane & ~1);
      if (h == 1) {
        float tot = (((from_lo + l0) + l1) + l2) + l3;
        for (int d = 8 * d8; d < a.dim; ++d) {
          const float e = qr[d] - cr[d];
          tot = tot + e * e;
        }
        cand[qi * cap + slot].y = __float_as_uint(tot);
      }
    }
    __syncthreads();

    // selection: a served query's candidate of rank r by (distance, centroid
    // index) goes to probe slot r < np (distances are >= +0, so their bits
    // order as the values do).  Wave w takes queries 8w .. 8w+7; lane l ranks
    // candidate r0 + l against all, read sixteen at a time (every lane the
    // same address; the padding keys never count) and compared from
    // registers.
    for (int t = 0; t < 32 / kW; ++t) {
      const int qi = wave * (32 / kW) + t;
      const uint32_t n = __builtin_amdgcn_readfirstlane(s_cnt[qi]);
      const uint4* __restrict__ cq2 = reinterpret_cast<const uint4*>(cand + qi * cap);
      const uint64_t qq = q0 + (uint64_t)qi;
      for (uint32_t r0 = 0; r0 < n; r0 += 64) {
        const uint32_t j = r0 + (uint32_t)lane;
        const uint2 me = j < n ? cand[qi * cap + j] : make_uint2(0xFFFFFFFFu, 0xFFFFFFFFu);
        const uint64_t key = ((uint64_t)me.y << 32) | me.x;
        uint32_t rank = 0;
        for (uint32_t c0 = 0; c0 < n; c0 += 16) {
          uint4 w[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) w[i] = cq2[c0 / 2 + i];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            rank += ((((uint64_t)w[i].y << 32) | w[i].x) < key) ? 1u : 0u;
            rank += ((((uint64_t)w[i].w << 32) | w[i].z) < key) ? 1u : 0u;
          }
        }
        if (j < n && rank < (uint32_t)a.np) {
          a.probes[qq * a.np + rank] = (int32_t)me.x;
          if (a.dists) a.dists[qq * a.np + rank] = __uint_as_float(me.y);
        }
      }
    }
  }
}

// One wave per screened query: the exact distance of each candidate in the
// reference's order (a lane per candidate: FMA lanes 0..7 over the 8-float
// chunks, lanes summed 0..7 in order, then the scalar tail), then each
// candidate's rank by (distance bits, centroid index) gives its probe slot
// (distances are >= +0, so their bits order as the values do).  Queries
// flagged by the screening kernel are left to the exact kernel.
__global__ __launch_bounds__(kT) void coarse16_rescore_kernel(C16Args a) {
  __shared__ __align__(16) float qrow[kT / 64][256];
  __shared__ uint2 keys[kT / 64][kMaxCap];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint64_t q = (uint64_t)blockIdx.x * (kT / 64) + wave;
  if (q >= a.nq) return;
  const uint32_t n = a.ncand[q];
  if (n == 0) return;  // flagged (its flag is set): the exact kernel serves it
  const int dim = a.dim;
  float* __restrict__ qr = qrow[wave];
  for (int d = lane; d < dim; d += 64) qr[d] = a.queries[q * (uint64_t)dim + d];
  __builtin_amdgcn_wave_barrier();
  const int d8 = dim / 8;
  for (uint32_t c0 = 0; c0 < n; c0 += 64) {
    const uint32_t c = c0 + (uint32_t)lane;
    const bool has = c < n;
    const uint32_t id = has ? a.cand[q * (uint64_t)a.cap + c] : 0u;
    const float* __restrict__ cr = a.centroids + (uint64_t)id * dim;
    float l[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) l[t] = 0.0f;
    // chunks of 8 floats: groups of four chunks (32 floats), the next
    // group's loads issued before the current group's products, then the
    // chunks left one at a time
    auto acc = [&](const v4f* x, int j0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const v4f y = *reinterpret_cast<const v4f*>(qr + 8 * j0 + 4 * u);
        const int t0 = 4 * (u & 1);
        const float e0 = y.x - x[u].x, e1 = y.y - x[u].y, e2 = y.z - x[u].z, e3 = y.w - x[u].w;
        l[t0] = __builtin_fmaf(e0, e0, l[t0]);
        l[t0 + 1] = __builtin_fmaf(e1, e1, l[t0 + 1]);
        l[t0 + 2] = __builtin_fmaf(e2, e2, l[t0 + 2]);
        l[t0 + 3] = __builtin_fmaf(e3, e3, l[t0 + 3]);
      }
    };
    auto load4 = [&](v4f* x, int j0) {
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const v4f*>(cr + 8 * j0 + 4 * u);
    };
    int j = 0;
    if (a.vec) {
      const int ng = d8 / 4;
      v4f xa[8], xb[8];
      if (ng > 0) load4(xa, 0);
      for (int g = 0; g < ng; g += 2) {
        if (g + 1 < ng) load4(xb, 4 * (g + 1));
        acc(xa, 4 * g);
        if (g + 1 < ng) {
          if (g + 2 < ng) load4(xa, 4 * (g + 2));
          acc(xb, 4 * (g + 1));
        }
      }
      j = 4 * ng;
      for (; j < d8; ++j) {
        const v4f x0 = *reinterpret_cast<const v4f*>(cr + 8 * j);
        const v4f x1 = *reinterpret_cast<const v4f*>(cr + 8 * j + 4);
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float e = qr[8 * j + t] - x[t];
          l[t] = __builtin_fmaf(e, e, l[t]);
        }
      }
    }
    for (; j < d8; ++j) {
      float x[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) x[t] = cr[8 * j + t];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float e = qr[8 * j + t] - x[t];
        l[t] = __builtin_fmaf(e, e, l[t]);
      }
    }
    float tot = l[0];
#pragma unroll
    for (int t = 1; t < 8; ++t) tot = tot + l[t];
    for (int d = 8 * d8; d < dim; ++d) {
      const float e = qr[d] - cr[d];
      tot = tot + e * e;
    }
    if (has) keys[wave][c] = make_uint2(id, __float_as_uint(tot));  // c < n <= cap <= kMaxCap
  }
  __builtin_amdgcn_wave_barrier();
  // ranks: every candidate against all n, read as LDS broadcasts
  const uint2* __restrict__ kw = keys[wave];
  for (uint32_t c0 = 0; c0 < n; c0 += 64) {
    const uint32_t c = c0 + (uint32_t)lane;
    const uint2 me = c < n ? kw[c] : make_uint2(0u, 0u);
    const uint64_t key = ((uint64_t)me.y << 32) | me.x;
    uint32_t rank = 0;
    for (uint32_t i = 0; i < n; ++i) {
      const uint2 o = kw[i];
      rank += ((((uint64_t)o.y << 32) | o.x) < key) ? 1u : 0u;
    }
    if (c < n && rank < (uint32_t)a.np) {
      a.probes[q * a.np + rank] = (int32_t)me.x;
      if (a.dists) a.dists[q * a.np + rank] = __uint_as_float(me.y);
    }
  }
}
}  // namespace

void Coarse16::build(const float* cen, uint32_t nlist, uint32_t dim, hipStream_t s) {
  ok_ = false;
  nlist_ = nlist;
  dim_ = dim;
  KC_ = (int)((dim + 15) / 16);
  if (dim == 0 || nlist == 0 || KC_ > 16) return;
  nblk_ = (uint32_t)cdiv(nlist, 32);
  stats_.reserve(2);
  const uint32_t zero[2] = {0, 0};
  FDB_HIP(hipMemcpyAsync(stats_.p, zero, sizeof(zero), hipMemcpyHostToDevice, s));
  const uint64_t n = (uint64_t)nlist * dim;
  hipLaunchKernelGGL(c16_stats_kernel, dim3((unsigned)std::min<uint64_t>(cdiv(n, kT), 1024)), dim3(kT), 0, s, cen, n,
                     stats_.p);
  FDB_HIP(hipGetLastError());
  uint32_t st[2] = {0, 0};
  FDB_HIP(hipMemcpyAsync(st, stats_.p, 4, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  if (st[0] >= 0x7F800000u) return;  // a non-finite component
  float mxv;
  std::memcpy(&mxv, &st[0], 4);
  xexp_ = 0;
  if (mxv > 0.0f) {
    int E;
    (void)std::frexp(mxv, &E);
    xexp_ = 13 - E;
  }
  if (xexp_ > 100 || xexp_ < -100) return;
  blocks_.reserve((uint64_t)nblk_ * KC_ * 64);
  cnp_.reserve((uint64_t)nblk_ * 32);
  hipLaunchKernelGGL(c16_blocks_kernel, dim3(nblk_), dim3(64 * KC_), 0, s, cen, nlist, (int)dim, KC_,
                     std::ldexp(1.0f, xexp_), blocks_.p, cnp_.p, stats_.p);
  FDB_HIP(hipGetLastError());
  FDB_HIP(hipMemcpyAsync(st, stats_.p, 8, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  float x2;
  std::memcpy(&x2, &st[1], 4);
  if (!(x2 <= 3.0e38f)) return;  // a norm fp32 cannot hold
  xnorm_ = std::sqrt(x2) * (1.0f + 0x1p-16f);
  // the reference's distance: dim squares, each rounded with its
  // difference, summed in at most dim steps
  screen_eps_coeffs(16 * KC_, (int)dim + 2, mxv, c_dot_, c_sq_, cabs_);
  ok_ = true;
}

void Coarse16::select(const float* d_qs, uint64_t nq, uint32_t np, const float* d_centroids, int32_t* probes,
                      float* dists, int* flags, hipStream_t s) {
  if (nq == 0) return;
  C16Args a{};
  a.queries = d_qs;
  a.nq = nq;
  a.dim = (int)dim_;
  a.vec = dim_ % 4 == 0 && (reinterpret_cast<uintptr_t>(d_centroids) & 15) == 0;
  a.centroids = d_centroids;
  a.nlist = nlist_;
  a.nblk = nblk_;
  a.blocks = blocks_.p;
  a.cnp = cnp_.p;
  a.xexp = xexp_;
  a.c_dot = c_dot_;
  a.c_sq = c_sq_;
  a.cabs = cabs_;
  a.xnorm = xnorm_;
  a.np = (int)np;
  // candidate slots per query: 1.5 np + 32 rounded up to 64 (the screened
  // candidates are the np nearest, those sharing a half-block with one of
  // them, and the few within 2 eps; a query with more is flagged)
  a.cap = (int)((3 * np / 2 + 32 + 63) / 64 * 64);
  if (a.cap > kMaxCap) throw Error(FDB_ERR_HIP, "coarse screening: nprobe above 64");
  a.probes = probes;
  a.dists = dists;
  a.flags = flags;
  cand_.reserve(nq * (uint64_t)a.cap);
  ncand_.reserve(nq);
  a.cand = cand_.p;
  a.ncand = ncand_.p;
  const size_t lds = (size_t)32 * (16 * KC_ + 4) * 4 + (size_t)32 * a.cap * 8;
  const bool m16 = np > 32;  // 8 M >= np kept minima per query
  // the kept minima ([32][8 M + 4] floats) are held in the candidate slots
  if ((8 * (m16 ? 16 : 8) + 4) * 4 > a.cap * 8) throw Error(FDB_ERR_HIP, "coarse screening: minima exceed the slots");
  void (*fn)(C16Args) = nullptr;
#define FDB_C16(K)                                          \
  case K:                                                   \
    fn = m16 ? coarse16_kernel<K, 16> : coarse16_kernel<K, 8>; \
    break;
  switch (KC_) {
    FDB_C16(1) FDB_C16(2) FDB_C16(3) FDB_C16(4) FDB_C16(5) FDB_C16(6) FDB_C16(7) FDB_C16(8)
    FDB_C16(9) FDB_C16(10) FDB_C16(11) FDB_C16(12) FDB_C16(13) FDB_C16(14) FDB_C16(15) FDB_C16(16)
  }
#undef FDB_C16
  if (!fn) throw Error(FDB_ERR_HIP, "no coarse screening kernel for this dimension");
  FDB_HIP(hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
  hipLaunchKernelGGL(fn, dim3((unsigned)cdiv(nq, 32)), dim3(kCT), lds, s, a);
  FDB_HIP(hipGetLastError());
  if (m16) {
    hipLaunchKernelGGL(coarse16_rescore_kernel, dim3((unsigned)cdiv(nq, kT / 64)), dim3(kT), 0, s, a);
    FDB_HIP(hipGetLastError());
  }
}

}  // namespace fdb
