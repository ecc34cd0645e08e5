// Full-precision search on gfx950: BruteForceIndex (src/index/brute_force.rs)
// and IVFIndex (src/index/ivf.rs).
//
// Every distance is computed in the reference's AVX2 operation order for its
// metric (src/distance/simd.rs:290-517): eight lane chains over elements
// i = l (mod 8) of the full 8-blocks (FMA for squared L2, dot and cosine;
// add of |a-b| for Manhattan), lanes summed left to right, then the scalar
// tail as separate operations; sqrt / negation / 1 - dot/sqrt(na*nb) last
// (src/distance/mod.rs:40-48).  Cosine takes the two norms from the same
// order, precomputed per row and per query.
#include "fdb_flat.hpp"

#include <algorithm>
#include <cstring>

#include "fdb_device.hpp"
#include "fdb_ivfpq.hpp"
#include "fdb_kernels.hpp"
#include "forgedb_hip.h"

namespace fdb {

namespace {

constexpr int kT = 256;
constexpr int kTQ = 4;        // queries per wave in the brute-force tile
constexpr int kQB = 4 * kTQ;  // queries per workgroup

template <int MET>
__device__ __forceinline__ float chain_step(float acc, float q, float x) {
  if constexpr (MET == FDB_METRIC_EUCLIDEAN || MET == FDB_METRIC_EUCLIDEAN_SQUARED) {
    const float d = q - x;
    return __builtin_fmaf(d, d, acc);
  } else if constexpr (MET == FDB_METRIC_COSINE || MET == FDB_METRIC_DOT_PRODUCT) {
    return __builtin_fmaf(q, x, acc);
  } else {
    return acc + __builtin_fabsf(q - x);
  }
}

template <int MET>
__device__ __forceinline__ float tail_step(float tot, float q, float x) {
  if constexpr (MET == FDB_METRIC_EUCLIDEAN || MET == FDB_METRIC_EUCLIDEAN_SQUARED) {
    const float d = q - x;
    return tot + d * d;
  } else if constexpr (MET == FDB_METRIC_COSINE || MET == FDB_METRIC_DOT_PRODUCT) {
    return tot + q * x;
  } else {
    return tot + __builtin_fabsf(q - x);
  }
}

template <int MET>
__device__ __forceinline__ float finish(float tot, float qn, float rn) {
  if constexpr (MET == FDB_METRIC_EUCLIDEAN) {
    return __builtin_sqrtf(tot);
  } else if constexpr (MET == FDB_METRIC_COSINE) {
    const float np = __builtin_sqrtf(qn * rn);
    return np == 0.0f ? 0.0f : 1.0f - tot / np;
  } else if constexpr (MET == FDB_METRIC_DOT_PRODUCT) {
    return -tot;
  } else {
    return tot;
  }
}

__device__ __forceinline__ int perm_row(int d, int dim) {
  const int d8 = dim / 8;
  return (d >= 8 * d8) ? d : (d % 8) * d8 + d / 8;
}

__global__ __launch_bounds__(kT) void transpose_rows_kernel(const float* __restrict__ rows, uint64_t n,
                                                            int dim, uint64_t ld,
                                                            float* __restrict__ out) {
  const uint64_t e = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (e >= ld * (uint64_t)dim) return;
  const uint64_t r = e / dim;
  const int d = (int)(e - r * dim);
  out[(uint64_t)perm_row(d, dim) * ld + r] = (r < n) ? rows[e] : 0.0f;
}

// reference-order sum of squares of one row (cosine norms)
__global__ __launch_bounds__(kT) void row_norms_kernel(const float* __restrict__ rows, uint64_t n,
                                                       int dim, float* __restrict__ out) {
  const uint64_t r = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (r >= n) return;
  const float* __restrict__ a = rows + r * dim;
  const int nb = dim / 8;
  float total = 0.0f;
  if (nb > 0) {
    float lane[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) lane[l] = 0.0f;
    for (int i = 0; i < nb; ++i)
#pragma unroll
      for (int l = 0; l < 8; ++l) lane[l] = __builtin_fmaf(a[8 * i + l], a[8 * i + l], lane[l]);
    total = lane[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) total = total + lane[l];
  }
  for (int i = 8 * nb; i < dim; ++i) total = total + a[i] * a[i];
  out[r] = total;
}

// Distances of TQ queries against 4 consecutive rows (one float4 per permuted
// dimension row) in reference order.  TQ == 4: the wave's 4 query values of a
// permuted row are a float4 at qw + row * kQB; TQ == 1: one value at qw[row].
// data: permuted rows with leading dimension ld, starting at column c.
template <int MET, int TQ>
__device__ __forceinline__ void tile_dist(const float* __restrict__ qw, const float* __restrict__ data,
                                          uint64_t ld, uint64_t c, int dim, float (&tot)[TQ][4]) {
  const int d8 = dim / 8;
  auto qload = [&](int row, float (&qa)[TQ]) {
    if constexpr (TQ == 4) {
      const float4 qv = *reinterpret_cast<const float4*>(qw + row * kQB);
      qa[0] = qv.x;
      qa[1] = qv.y;
      qa[2] = qv.z;
      qa[3] = qv.w;
    } else {
      qa[0] = qw[row];
    }
  };
#pragma unroll
  for (int t = 0; t < TQ; ++t)
#pragma unroll
    for (int u = 0; u < 4; ++u) tot[t][u] = 0.0f;
#pragma unroll 1
  for (int l = 0; l < 8 && d8 > 0; ++l) {
    float ch[TQ][4];
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) ch[t][u] = 0.0f;
#pragma unroll 4
    for (int i = 0; i < d8; ++i) {
      const int row = l * d8 + i;
      const float4 xv = *reinterpret_cast<const float4*>(data + (uint64_t)row * ld + c);
      const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
      float qa[TQ];
      qload(row, qa);
#pragma unroll
      for (int t = 0; t < TQ; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) ch[t][u] = chain_step<MET>(ch[t][u], qa[t], xa[u]);
    }
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) tot[t][u] = (l == 0) ? ch[t][u] : tot[t][u] + ch[t][u];
  }
  for (int row = 8 * d8; row < dim; ++row) {
    const float4 xv = *reinterpret_cast<const float4*>(data + (uint64_t)row * ld + c);
    const float xa[4] = {xv.x, xv.y, xv.z, xv.w};
    float qa[TQ];
    qload(row, qa);
#pragma unroll
    for (int t = 0; t < TQ; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) tot[t][u] = tail_step<MET>(tot[t][u], qa[t], xa[u]);
  }
}

// ---------------------------------------------------------------------------
// Brute force, partial top-k per (16-query tile, row chunk).  Each wave owns
// 4 queries, each lane 4 adjacent rows; the row chunk is swept 256 rows at a
// time and every distance is offered to the wave's per-query WaveTopK.
// ---------------------------------------------------------------------------
template <int MET, int R>
__global__ __launch_bounds__(kT) void flat_topk_kernel(FlatTopkArgs a) {
  extern __shared__ float qsT[];  // [dim][kQB], rows permuted
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t chunk = blockIdx.x;
  const uint64_t q0 = (uint64_t)blockIdx.y * kQB;
  const int dim = a.dim;
  if (a.flags) {  // re-run only tiles holding a flagged query (uniform exit)
    bool any = false;
    for (int t = 0; t < kQB; ++t) any |= (q0 + t < a.nq) && a.flags[q0 + t] != 0;
    if (!any) return;
  }
  for (int e = tid; e < kQB * dim; e += kT) {
    const int qq = e / dim;
    const int d = e - qq * dim;
    qsT[perm_row(d, dim) * kQB + qq] = (q0 + qq < a.nq) ? a.queries[(q0 + qq) * (uint64_t)dim + d] : 0.0f;
  }
  WaveTopK<R> tk[kTQ];
  float qn[kTQ];
#pragma unroll
  for (int t = 0; t < kTQ; ++t) {
    tk[t].init(a.k);
    const uint64_t q = q0 + wave * kTQ + t;
    qn[t] = (MET == FDB_METRIC_COSINE && q < a.nq) ? a.q_norm[q] : 0.0f;
  }
  __syncthreads();
  const float* __restrict__ qw = qsT + wave * kTQ;
  const uint64_t r0 = (uint64_t)chunk * a.chunk_rows;
  const uint64_t r1 = std::min<uint64_t>(a.n, r0 + a.chunk_rows);
  for (uint64_t base = r0; base < r1; base += 256) {
    const uint64_t c = base + 4 * (uint64_t)lane;  // c + 3 < ld: ld is a multiple of 256
    float tot[kTQ][4];
    tile_dist<MET, kTQ>(qw, a.dataT, a.ld, c, dim, tot);
    float rn[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (MET == FDB_METRIC_COSINE) {
#pragma unroll
      for (int u = 0; u < 4; ++u) rn[u] = (c + u < r1) ? a.row_norm[c + u] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool in = c + u < r1;
#pragma unroll
      for (int t = 0; t < kTQ; ++t) {
        const float dv = finish<MET>(tot[t][u], qn[t], rn[u]);
        tk[t].offer(in ? dv : f_inf(), in ? (uint32_t)(c + u) : kNoPos);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kTQ; ++t) {
    const uint64_t q = q0 + wave * kTQ + t;
    if (q >= a.nq) continue;
    const uint64_t o = (q * a.nchunks + chunk) * (uint64_t)a.k;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int s = r * 64 + lane;
      if (s < a.k) {
        a.part_d[o + s] = tk[t].d[r];
        a.part_key[o + s] = tk[t].p[r];
      }
    }
  }
}

// One wave per query: the k smallest (distance, key) of its partial lists.
template <int R>
__global__ __launch_bounds__(64) void merge_parts_kernel(const float* __restrict__ pd,
                                                         const uint32_t* __restrict__ pk, uint64_t nq,
                                                         uint32_t nparts, int k,
                                                         const uint64_t* __restrict__ ids,
                                                         uint64_t* __restrict__ out_ids,
                                                         float* __restrict__ out_d,
                                                         uint32_t* __restrict__ out_c,
                                                         const int* __restrict__ flags) {
  const uint64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  if (flags && flags[q] == 0) return;
  WaveTopK<R> tk;
  tk.init(k);
  const uint64_t total = (uint64_t)nparts * k;
  for (uint64_t b = 0; b < total; b += 64) {
    const uint64_t e = b + lane;
    float d = f_inf();
    uint32_t key = kNoPos;
    if (e < total) {
      d = pd[q * total + e];
      key = pk[q * total + e];
      if (key == kNoPos) d = f_inf();
    }
    tk.offer(d, key);
  }
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = r * 64 + lane;
    const bool valid = s < k && tk.p[r] != kNoPos;
    count += (uint32_t)__popcll(__ballot(valid));
    if (s < k) {
      out_ids[q * k + s] = valid ? (ids ? ids[tk.p[r]] : (uint64_t)tk.p[r]) : ~0ull;
      out_d[q * k + s] = valid ? tk.d[r] : f_inf();
    }
  }
  if (lane == 0) out_c[q] = count;
}

// ---------------------------------------------------------------------------
// IVF-flat scan.  One workgroup (4 waves) per query; probed list j goes to
// wave j % 4.  List p is a block [dim][lld_p] of permuted dimension rows;
// each lane takes 4 adjacent rows, so every load is a float4 and the query is
// a wave-uniform LDS broadcast.  Keys are list-order row positions.
// ---------------------------------------------------------------------------
template <int MET, int R>
__global__ __launch_bounds__(kT) void ivf_flat_scan_kernel(IvfFlatScanArgs a) {
  extern __shared__ float qp[];  // [dim] permuted; then the merge buffer
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t q = blockIdx.x;
  if (a.flags && a.flags[q] == 0) return;  // settled by screening
  const int dim = a.dim;
  for (int d = tid; d < dim; d += kT) qp[perm_row(d, dim)] = a.queries[q * dim + d];
  const float qn = (MET == FDB_METRIC_COSINE) ? a.q_norm[q] : 0.0f;
  WaveTopK<R> tk;
  tk.init(a.k);
  __syncthreads();
  const int32_t* __restrict__ pr = a.probes + q * (uint64_t)a.np;
  for (int j = wave; j < a.np; j += 4) {
    const int p = pr[j];
    if (p < 0 || p >= a.nlist) continue;  // wave-uniform
    const uint32_t rs = a.row_off[p];
    const uint32_t len = a.row_off[p + 1] - rs;
    const uint64_t lld = (len + 3) / 4 * 4;
    const float* __restrict__ blk = a.data + a.boff[p];
    for (uint32_t base = 0; base < len; base += 256) {
      uint64_t c = base + 4 * (uint64_t)lane;
      const bool any = c < lld;
      if (!any) c = 0;  // re-read the first rows; nothing is offered
      float tot[1][4];
      tile_dist<MET, 1>(qp, blk, lld, c, dim, tot);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool in = any && c + u < len;
        float dv = f_inf();
        if (in) dv = finish<MET>(tot[0][u], qn, MET == FDB_METRIC_COSINE ? a.row_norm[rs + c + u] : 0.0f);
        tk.offer(dv, in ? rs + (uint32_t)(c + u) : kNoPos);
      }
    }
  }
  // merge the 4 wave lists in wave 0 (the query copy is no longer needed)
  __syncthreads();
  float* md = qp;
  uint32_t* mk = reinterpret_cast<uint32_t*>(qp + 4 * 64 * R);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    md[wave * 64 * R + r * 64 + lane] = tk.d[r];
    mk[wave * 64 * R + r * 64 + lane] = tk.p[r];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < 4; ++w)
#pragma unroll
    for (int r = 0; r < R; ++r) tk.offer(md[w * 64 * R + r * 64 + lane], mk[w * 64 * R + r * 64 + lane]);
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

// ---------------------------------------------------------------------------
// MFMA screening for dot product, cosine and (squared) Euclidean.
//
// mfma_screen_kernel: approximate distances from v_mfma_f32_32x32x2f32
// (query tile 32 x dim times 32 rows per wave, so 128 rows per workgroup
// step), turned into the metric's value with exact norms, and the K' = 64*RS
// smallest per query kept in wave-resident WaveTopK lists (each wave owns 8
// of the 32 queries).  The product sums the dimensions in some order of the
// matrix unit's choosing, so it differs from the reference's order by at most
// eps (see screen_eps); the rescore kernel computes exact distances for the
// K' candidates and checks that no row outside them can enter the top k.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kSQ = 32;    // queries per screening workgroup
constexpr int kSRows = 128;  // rows per workgroup step

// Reference-order distance of one query (LDS, natural order) to one row
// (global, natural order), computed by a single lane.
template <int MET>
__device__ __forceinline__ float exact_lane(const float* __restrict__ q, const float* __restrict__ x,
                                            int dim, float qn, float rn) {
  const int d8 = dim / 8;
  float total = 0.0f;
  if (d8 > 0) {
    float ch[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) ch[l] = 0.0f;
    for (int i = 0; i < d8; ++i) {
      const float4 x0 = *reinterpret_cast<const float4*>(x + 8 * i);
      const float4 x1 = *reinterpret_cast<const float4*>(x + 8 * i + 4);
      const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
      for (int l = 0; l < 8; ++l) ch[l] = chain_step<MET>(ch[l], q[8 * i + l], xv[l]);
    }
    total = ch[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) total = total + ch[l];
  }
  for (int i = 8 * d8; i < dim; ++i) total = tail_step<MET>(total, q[i], x[i]);
  return finish<MET>(total, qn, rn);
}

// Screening value: the metric's distance (squared for Euclidean) from an
// approximate dot product s.
template <int MET>
__device__ __forceinline__ float screen_value(float s, float qn, float rn) {
  if constexpr (MET == FDB_METRIC_DOT_PRODUCT) {
    return -s;
  } else if constexpr (MET == FDB_METRIC_COSINE) {
    const float np = __builtin_sqrtf(qn * rn);
    return np == 0.0f ? 0.0f : 1.0f - s / np;
  } else {
    return __builtin_fmaf(-2.0f, s, qn + rn);
  }
}

// Bound on |screen value - reference value| for one query (squared domain
// for Euclidean), with u = 2^-24 and g = dim*u/(1 - dim*u) the classic
// bound for a dim-term float sum:
//   dot:     both sums within g*sum|q_i x_i| <= g*|q|*max|x| of the exact dot
//   cosine:  the same over np ~ |q||x|, plus the division and 1 - x roundings
//   L2^2:    norms and dot each within g of their magnitudes; the
//            reference's sum of squares within (g + 3u) of the exact value
// with 10% slack and a floor for flushed denormal products.
__device__ __forceinline__ float screen_eps(int met, int dim, float qn, float rnmax) {
  const float u = 5.9604645e-8f;
  const float g = dim * u / (1.0f - dim * u);
  if (met == FDB_METRIC_DOT_PRODUCT) return 2.2f * g * __builtin_sqrtf(qn) * __builtin_sqrtf(rnmax) + 1e-30f;
  if (met == FDB_METRIC_COSINE) return 2.2f * g + 16.0f * u + 1e-30f;
  return (4.4f * g + 12.0f * u) * (qn + rnmax) + 1e-30f;
}

// The same bound for screening values from the fp16 product
// (v_mfma_f32_32x32x16_f16).  Rows and queries (for cosine: divided by
// their norms first) are scaled by powers of two so that their largest
// component lies in [2^13, 2^14) and rounded to fp16: each component is
// then off by at most uh = 2^-11 relative plus 2^-27 of the vector's
// largest component (values below the smallest fp16 normal, even if
// flushed).  The products of fp16 values are exact in fp32 and their sum is
// within g2 = dim*2u/(1 - dim*2u) of the exact sum in any order, rounded or
// truncated.  With h = 2uh + uh^2 + eta + 1.002*g2*(1 + eta), eta =
// 2.002*2^-27*sqrt(dim) + dim*2^-54:
//   dot:     (h + g) |q||x|, g for the reference's own sum
//   cosine:  h + g + 7u for the division by the norms, then the fp32
//            screen's 2.2g + 16u (both roundings of 1 - x and the
//            reference's cosine)
//   L2^2:    (h + 4g + 9u) (qn + rnmax): the product as for dot, the norms,
//            the three roundings of qn + rn - 2s and the reference's sum of
//            squares
// with 10% slack and a floor for products and sums near the fp32 underflow.
__device__ __forceinline__ float screen16_eps(int met, int dim, float qn, float rnmax) {
  const float u = 5.9604645e-8f;
  const float uh = 4.8828125e-4f;
  const float g = dim * u / (1.0f - dim * u);
  const float g2 = dim * 2.0f * u / (1.0f - dim * 2.0f * u);
  const float eta = 2.002f * 7.4505806e-9f * __builtin_sqrtf((float)dim) + dim * 5.551115e-17f;
  const float h = 2.0f * uh + uh * uh + eta + 1.002f * g2 * (1.0f + eta);
  if (met == FDB_METRIC_DOT_PRODUCT)
    return 1.1f * (h + g) * __builtin_sqrtf(qn) * __builtin_sqrtf(rnmax) + 1e-30f;
  if (met == FDB_METRIC_COSINE) return 1.1f * (h + 3.2f * g + 23.0f * u) + 1e-30f;
  return 1.1f * (h + 4.0f * g + 9.0f * u) * (qn + rnmax) + 1e-30f;
}

// IVF fp16 screening (fdb_ivf16.hip): rows and query scaled by the same 2^e
// and rounded to fp16 (uh = 2^-11 relative, values below 2^-14 * 2^-e off by
// at most eta = 2^-14 * 2^-e), differences rounded to fp16, squared (or
// taken absolute) exactly and summed in fp32 (within g2 = D*2u/(1 - D*2u)).
// Each component's screening difference is then within
//   E_i = uh (1 + uh) (|q_i| + |x_i| + |d_i|) + 3.01 eta
// of d_i = q_i - x_i.  The error grows with the row's own distance, so the
// check is monotone: with Dk the k-th reference value, Dp = Dk / (1 - g -
// 2.01u) bounds the exact value of every row whose reference value is at
// most Dk, and such a row screens at most
//   L2^2: (1 + g2) (Dp + 1.1 (2 uh (1 + uh) (A + s) s + 6.02 eta sqrt(D) s
//                             + 3 uh^2 (A + s)^2 + 20 D eta^2)),
//         s = sqrt(Dp), A = |q| + max|x|
//   L1:   (1 + g2) (Lp + 1.1 (uh (1 + uh) (|q|_1 + max|x|_1 + Lp) + 3.01 D eta))
// A screened list whose K'-th value exceeds that leaves out no such row.
__device__ __forceinline__ float ivf16_bound(bool l1, float vk, float qmag, float xmag, int xexp, int dim) {
  const float u = 5.9604645e-8f;
  const float uh = 4.8828125e-4f;
  const float g = dim * u / (1.0f - dim * u);
  const float g2 = dim * 2.0f * u / (1.0f - dim * 2.0f * u);
  const float eta = ldexpf(1.0f, -14 - xexp);
  if (l1) {
    const float lp = vk / (1.0f - g - 1.01f * u);
    const float err = uh * (1.0f + uh) * (qmag + xmag + lp) + 3.01f * dim * eta;
    return (1.0f + g2) * (lp + 1.1f * err) * 1.0001f + 1e-30f;
  }
  const float dp = vk / (1.0f - g - 2.01f * u);
  const float s = __builtin_sqrtf(dp);
  const float A = qmag + xmag;
  const float err = 2.0f * uh * (1.0f + uh) * (A + s) * s + 6.02f * eta * __builtin_sqrtf((float)dim) * s +
                    3.0f * uh * uh * (A + s) * (A + s) + 20.0f * dim * eta * eta;
  return (1.0f + g2) * (dp + 1.1f * err) * 1.0001f + 1e-30f;
}

template <int MET, int RS>
__global__ __launch_bounds__(kT) void mfma_screen_kernel(ScreenArgs a) {
  extern __shared__ float sm[];
  const int dim = a.dim;
  float* qT = sm;                     // [dim][kSQ], dimension rows permuted as dataT
  float* S = sm + dim * kSQ;          // [kSQ][kSRows] screening values of one step
  float* qn_s = S + kSQ * kSRows;     // [kSQ]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t q0 = (uint64_t)blockIdx.x * kSQ;
  const uint32_t chunk = blockIdx.y;
  for (int e = tid; e < kSQ * dim; e += kT) {
    const int qq = e / dim;
    const int d = e - qq * dim;
    qT[perm_row(d, dim) * kSQ + qq] = (q0 + qq < a.nq) ? a.queries[(q0 + qq) * (uint64_t)dim + d] : 0.0f;
  }
  if (tid < kSQ) qn_s[tid] = (q0 + tid < a.nq) ? a.q_norm[q0 + tid] : 0.0f;
  WaveTopK<RS> tk[kSQ / 4];
#pragma unroll
  for (int t = 0; t < kSQ / 4; ++t) tk[t].init(a.kp);
  __syncthreads();
  const int half = lane >> 5;
  const int col = lane & 31;
  const int kh = dim >> 1;  // lanes of half h take dimension rows h*kh .. h*kh+kh-1
  const float* __restrict__ ap = qT + half * kh * kSQ + col;
  const uint64_t r0 = (uint64_t)chunk * a.chunk_rows;
  const uint64_t r1 = std::min<uint64_t>(a.n, r0 + a.chunk_rows);
  for (uint64_t base = r0; base < r1; base += kSRows) {
    const uint64_t row = base + wave * 32 + col;  // < ld: base < n, ld a multiple of 256
    const float* __restrict__ bp = a.dataT + (uint64_t)half * kh * a.ld + row;
    v16f acc = {};
    int j = 0;
    for (; j + 8 <= kh; j += 8) {  // 8 row loads in flight, then 8 products
      float av[8], bv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        bv[u] = bp[(uint64_t)(j + u) * a.ld];
        av[u] = ap[(j + u) * kSQ];
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[u], bv[u], acc, 0, 0, 0);
    }
    for (; j < kh; ++j)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(ap[j * kSQ], bp[(uint64_t)j * a.ld], acc, 0, 0, 0);
    const bool in = row < r1;
    const float rn = in ? a.row_norm[row] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = 8 * (r >> 2) + 4 * half + (r & 3);  // D[qi][col] lives in register r
      const float v = screen_value<MET>(acc[r], qn_s[qi], rn);
      S[qi * kSRows + wave * 32 + col] = in ? v : f_inf();
    }
    __syncthreads();
#pragma unroll
    for (int t = 0; t < kSQ / 4; ++t) {
      const int qi = wave * (kSQ / 4) + t;
      if (q0 + qi >= a.nq) break;  // padding queries of the last tile
#pragma unroll
      for (int h2 = 0; h2 < kSRows / 64; ++h2) {
        const uint64_t key = base + h2 * 64 + lane;
        const bool ok = key < r1;
        tk[t].offer(ok ? S[qi * kSRows + h2 * 64 + lane] : f_inf(), ok ? (uint32_t)key : kNoPos);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int t = 0; t < kSQ / 4; ++t) {
    const uint64_t q = q0 + wave * (kSQ / 4) + t;
    if (q >= a.nq) continue;
    const uint64_t o = (q * a.nchunks + chunk) * (uint64_t)a.kp;
#pragma unroll
    for (int r = 0; r < RS; ++r) {
      a.part_d[o + r * 64 + lane] = tk[t].d[r];
      a.part_key[o + r * 64 + lane] = tk[t].p[r];
    }
  }
}

// One wave per query: exact reference-order distances of its K' = 64*RS
// screened candidates, their k smallest (WaveTopK<RK>), and the check that
// the candidates hold the exact top k: with a' the K'-th screening value
// (every other row screens at a' or above, so its exact distance is at least
// a' - eps), the list is final when a' - eps exceeds the k-th exact distance
// (for Euclidean: the k-th squared distance times 1 + 8u, so that no
// square root can round onto it).  Otherwise the query is flagged for the
// exact scan.
template <int MET, int RS, int RK>
__global__ __launch_bounds__(64) void rescore_kernel(RescoreArgs a) {
  extern __shared__ float qv[];  // [dim]
  const uint64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  const int dim = a.dim;
  for (int d = lane; d < dim; d += 64) qv[d] = a.queries[q * dim + d];
  __syncthreads();
  const int kp = 64 * RS;
  const uint32_t cnt0 = a.cand_counts[q];
  const bool forced = cnt0 == kForceExact;
  const uint32_t cnt = forced ? 0u : cnt0;
  const float qn = a.q_norm[q];
  constexpr int EM = (MET == FDB_METRIC_EUCLIDEAN) ? FDB_METRIC_EUCLIDEAN_SQUARED : MET;
  WaveTopK<RK> tk;
  tk.init(a.k);
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const uint32_t s = r * 64 + lane;
    const bool valid = s < cnt;
    const uint32_t key = valid ? (uint32_t)a.cand_keys[q * kp + s] : kNoPos;
    float e = f_inf();
    if (valid)
      e = exact_lane<MET>(qv, a.rows + (uint64_t)key * dim, dim, qn,
                          MET == FDB_METRIC_COSINE ? a.row_norm[key] : 0.0f);
    tk.offer(e, key);
  }
  const uint32_t kk = (uint32_t)a.k < cnt ? (uint32_t)a.k : cnt;
  bool ok = !forced;
  // with a threshold bound, fewer candidates than the top k needs is a miss
  if (a.bkind == kBoundH16 && (uint64_t)kk < ((uint64_t)a.k < a.n ? (uint64_t)a.k : a.n)) ok = false;
  // without one (all other rows screen above the K'-th candidate), fewer
  // than K' candidates means every row is a candidate
  const bool check = a.bkind == kBoundH16 || (cnt >= (uint32_t)kp && (a.bkind == kBoundF32 || a.abound[q] < f_inf()));
  if (ok && kk > 0 && check) {
    const float aK = a.bkind == kBoundF32 ? a.cand_d[q * kp + kp - 1] : a.abound[q];
    const int s = (int)kk - 1;
    // the k-th exact pair, in the screening domain
    float v = tk.d[0];
    uint32_t w = tk.p[0];
#pragma unroll
    for (int r = 1; r < RK; ++r) {
      const bool sel = r <= (s >> 6);
      v = sel ? tk.d[r] : v;
      w = sel ? tk.p[r] : w;
    }
    if constexpr (MET == FDB_METRIC_EUCLIDEAN) {
      const uint32_t wk = readlane_u(w, s & 63);
      float e2 = 0.0f;
      if (lane == (s & 63)) e2 = exact_lane<EM>(qv, a.rows + (uint64_t)wk * dim, dim, qn, 0.0f);
      v = readlane_f(e2, s & 63) * (1.0f + 8.0f * 5.9604645e-8f);
    } else {
      v = readlane_f(v, s & 63);
    }
    if (a.bkind == kBoundIvf16) {
      float qmag = 0.0f;  // |q|_1 for Manhattan, |q|_2 otherwise
      if constexpr (MET == FDB_METRIC_MANHATTAN) {
        for (int d = lane; d < dim; d += 64) qmag += __builtin_fabsf(qv[d]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) qmag += __shfl_xor(qmag, off);
        qmag *= 1.0f + (float)dim * 5.9604645e-8f;
      } else {
        qmag = __builtin_sqrtf(qn) * (1.0f + (float)dim * 5.9604645e-8f);
      }
      ok = aK > ivf16_bound(MET == FDB_METRIC_MANHATTAN, v, qmag, a.xmag, a.xexp, dim);
    } else {
      const float eps = a.bkind == kBoundH16 ? screen16_eps(MET, dim, qn, a.rnmax) : screen_eps(MET, dim, qn, a.rnmax);
      ok = aK - eps > v;
    }
  }
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < RK; ++r) {
    const int s = r * 64 + lane;
    const bool valid = s < a.k && tk.p[r] != kNoPos;
    count += (uint32_t)__popcll(__ballot(valid));
    if (s < a.k) {
      a.out_ids[q * a.k + s] = valid ? (a.ids ? a.ids[tk.p[r]] : (uint64_t)tk.p[r]) : ~0ull;
      a.out_d[q * a.k + s] = valid ? tk.d[r] : f_inf();
    }
  }
  if (lane == 0) {
    a.out_counts[q] = count;
    a.flags[q] = ok ? 0 : 1;
    if (!ok) atomicAdd(a.fallbacks, 1u);
  }
}

int regs_k(int k) {
  int r = (k + 63) / 64, p = 1;
  while (p < r) p <<= 1;
  return p;
}

template <int MET>
void* pick_flat(int R) {
  switch (R) {
    case 1: return (void*)flat_topk_kernel<MET, 1>;
    case 2: return (void*)flat_topk_kernel<MET, 2>;
    case 4: return (void*)flat_topk_kernel<MET, 4>;
    case 8: return (void*)flat_topk_kernel<MET, 8>;
    case 16: return (void*)flat_topk_kernel<MET, 16>;
  }
  return nullptr;
}

template <int MET>
void* pick_ivf(int R) {
  switch (R) {
    case 1: return (void*)ivf_flat_scan_kernel<MET, 1>;
    case 2: return (void*)ivf_flat_scan_kernel<MET, 2>;
    case 4: return (void*)ivf_flat_scan_kernel<MET, 4>;
    case 8: return (void*)ivf_flat_scan_kernel<MET, 8>;
    case 16: return (void*)ivf_flat_scan_kernel<MET, 16>;
  }
  return nullptr;
}

void* pick_metric(int metric, int R, bool ivf) {
  switch (metric) {
    case FDB_METRIC_EUCLIDEAN: return ivf ? pick_ivf<FDB_METRIC_EUCLIDEAN>(R) : pick_flat<FDB_METRIC_EUCLIDEAN>(R);
    case FDB_METRIC_EUCLIDEAN_SQUARED:
      return ivf ? pick_ivf<FDB_METRIC_EUCLIDEAN_SQUARED>(R) : pick_flat<FDB_METRIC_EUCLIDEAN_SQUARED>(R);
    case FDB_METRIC_COSINE: return ivf ? pick_ivf<FDB_METRIC_COSINE>(R) : pick_flat<FDB_METRIC_COSINE>(R);
    case FDB_METRIC_DOT_PRODUCT: return ivf ? pick_ivf<FDB_METRIC_DOT_PRODUCT>(R) : pick_flat<FDB_METRIC_DOT_PRODUCT>(R);
    case FDB_METRIC_MANHATTAN: return ivf ? pick_ivf<FDB_METRIC_MANHATTAN>(R) : pick_flat<FDB_METRIC_MANHATTAN>(R);
  }
  return nullptr;
}

template <int MET>
void* pick_screen(int RS) {
  return RS == 1 ? (void*)mfma_screen_kernel<MET, 1> : (void*)mfma_screen_kernel<MET, 2>;
}

template <int MET>
void* pick_rescore(int RS, int RK) {
  if (RS == 1) return (void*)rescore_kernel<MET, 1, 1>;
  return RK == 1 ? (void*)rescore_kernel<MET, 2, 1> : (void*)rescore_kernel<MET, 2, 2>;
}

unsigned nblocks(uint64_t n, unsigned t) { return (unsigned)((n + t - 1) / t); }

__global__ void clear_u32(uint32_t* p) { *p = 0; }

__global__ void fill_empty(uint64_t n, uint32_t k, uint64_t* ids, float* d, uint32_t* c) {
  const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n * k) {
    ids[e] = ~0ull;
    d[e] = f_inf();
  }
  if (e < n) c[e] = 0;
}

__global__ void iota_probes(uint64_t nq, uint32_t np, int32_t* probes) {
  const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < nq * np) probes[e] = (int32_t)(e % np);
}

__global__ void clear_flag(int* p) { *p = 0; }

}  // namespace

hipError_t launch_transpose_rows(const float* rows, uint64_t n, int dim, uint64_t ld, float* out,
                                 hipStream_t s) {
  const uint64_t total = ld * (uint64_t)dim;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(transpose_rows_kernel, dim3(nblocks(total, kT)), dim3(kT), 0, s, rows, n, dim, ld, out);
  return hipGetLastError();
}

hipError_t launch_row_norms(const float* rows, uint64_t n, int dim, float* out, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(row_norms_kernel, dim3(nblocks(n, kT)), dim3(kT), 0, s, rows, n, dim, out);
  return hipGetLastError();
}

hipError_t launch_flat_topk(const FlatTopkArgs& a, hipStream_t s) {
  if (a.nq == 0 || a.nchunks == 0) return hipSuccess;
  if (a.k <= 0 || a.k > 1024 || a.dim <= 0 || a.dim > 2048 || a.ld % 256 != 0) return hipErrorInvalidValue;
  void* fn = pick_metric(a.metric, regs_k(a.k), false);
  if (!fn) return hipErrorInvalidValue;
  const size_t lds = sizeof(float) * (size_t)kQB * a.dim;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  void* args[] = {(void*)&a};
  return hipLaunchKernel(fn, dim3(a.nchunks, (unsigned)((a.nq + kQB - 1) / kQB)), dim3(kT), args, lds, s);
}

hipError_t launch_merge_parts(const float* pd, const uint32_t* pk, uint64_t nq, uint32_t nparts, int k,
                              const uint64_t* ids, uint64_t* out_ids, float* out_d, uint32_t* out_c,
                              hipStream_t s, const int* flags) {
  if (nq == 0) return hipSuccess;
#define FDB_MP(R)                                                                                 \
  hipLaunchKernelGGL(merge_parts_kernel<R>, dim3((unsigned)nq), dim3(64), 0, s, pd, pk, nq, nparts, \
                     k, ids, out_ids, out_d, out_c, flags);                                      \
  break;
  switch (regs_k(k)) {
    case 1: FDB_MP(1)
    case 2: FDB_MP(2)
    case 4: FDB_MP(4)
    case 8: FDB_MP(8)
    case 16: FDB_MP(16)
    default: return hipErrorInvalidValue;
  }
#undef FDB_MP
  return hipGetLastError();
}

hipError_t launch_mfma_screen(const ScreenArgs& a, hipStream_t s) {
  if (a.nq == 0 || a.nchunks == 0) return hipSuccess;
  if ((a.kp != 64 && a.kp != 128) || a.dim <= 0 || a.dim > 512 || a.dim % 4 != 0 || a.ld % 256 != 0 ||
      a.chunk_rows % 256 != 0)
    return hipErrorInvalidValue;
  const int RS = a.kp / 64;
  void* fn = nullptr;
  switch (a.metric) {
    case FDB_METRIC_EUCLIDEAN:
    case FDB_METRIC_EUCLIDEAN_SQUARED: fn = pick_screen<FDB_METRIC_EUCLIDEAN_SQUARED>(RS); break;
    case FDB_METRIC_COSINE: fn = pick_screen<FDB_METRIC_COSINE>(RS); break;
    case FDB_METRIC_DOT_PRODUCT: fn = pick_screen<FDB_METRIC_DOT_PRODUCT>(RS); break;
    default: return hipErrorInvalidValue;
  }
  const size_t lds = sizeof(float) * ((size_t)a.dim * kSQ + kSQ * kSRows + kSQ);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  void* args[] = {(void*)&a};
  return hipLaunchKernel(fn, dim3((unsigned)((a.nq + kSQ - 1) / kSQ), a.nchunks), dim3(kT), args, lds, s);
}

hipError_t launch_rescore(const RescoreArgs& a, uint64_t nq, hipStream_t s) {
  if (nq == 0) return hipSuccess;
  if ((a.kp != 64 && a.kp != 128) || a.k <= 0 || a.k > a.kp || a.dim <= 0 || a.dim > 512 ||
      a.dim % 4 != 0)
    return hipErrorInvalidValue;
  const int RS = a.kp / 64, RK = regs_k(a.k);
  void* fn = nullptr;
  switch (a.metric) {
    case FDB_METRIC_EUCLIDEAN: fn = pick_rescore<FDB_METRIC_EUCLIDEAN>(RS, RK); break;
    case FDB_METRIC_EUCLIDEAN_SQUARED: fn = pick_rescore<FDB_METRIC_EUCLIDEAN_SQUARED>(RS, RK); break;
    case FDB_METRIC_COSINE: fn = pick_rescore<FDB_METRIC_COSINE>(RS, RK); break;
    case FDB_METRIC_DOT_PRODUCT: fn = pick_rescore<FDB_METRIC_DOT_PRODUCT>(RS, RK); break;
    case FDB_METRIC_MANHATTAN:
      if (a.bkind != kBoundIvf16) return hipErrorInvalidValue;
      fn = pick_rescore<FDB_METRIC_MANHATTAN>(RS, RK);
      break;
    default: return hipErrorInvalidValue;
  }
  void* args[] = {(void*)&a};
  return hipLaunchKernel(fn, dim3((unsigned)nq), dim3(64), args, sizeof(float) * a.dim, s);
}

hipError_t launch_ivf_flat_scan(const IvfFlatScanArgs& a, hipStream_t s) {
  if (a.nq == 0) return hipSuccess;
  if (a.k <= 0 || a.k > 1024 || a.dim <= 0 || a.dim > 2048) return hipErrorInvalidValue;
  const int R = regs_k(a.k);
  void* fn = pick_metric(a.metric, R, true);
  if (!fn) return hipErrorInvalidValue;
  const size_t lds = std::max(sizeof(float) * (size_t)a.dim, (size_t)4 * 64 * R * 8);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
  }
  void* args[] = {(void*)&a};
  return hipLaunchKernel(fn, dim3((unsigned)a.nq), dim3(kT), args, lds, s);
}

// ===========================================================================
// BruteForceIndex
// ===========================================================================
BruteForceIndex::BruteForceIndex(uint32_t metric) : metric_(metric) {
  if (metric > 4) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown metric");
  FDB_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  for (auto& e : ev_) FDB_HIP(hipEventCreate(&e));
}

void BruteForceIndex::add(const float* rows, const uint64_t* ids, uint64_t n, uint32_t dim) {
  if (n == 0) return;
  if (!rows) throw Error(FDB_ERR_INVALID_ARGUMENT, "null rows");
  if (dim == 0) throw Error(FDB_ERR_INVALID_ARGUMENT, "dim must be positive");
  std::lock_guard<std::mutex> g(mu_);
  if (!h_ids_.empty() && dim != dim_)
    throw Error(FDB_ERR_DIMENSION_MISMATCH, "vector dimension does not match the index");
  if (dim > 2048) throw Error(FDB_ERR_UNSUPPORTED, "dim above 2048");
  if (h_ids_.size() + n >= 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "more than 2^32-2 rows");
  dim_ = dim;
  const uint64_t base = h_ids_.size();
  h_rows_.insert(h_rows_.end(), rows, rows + n * dim);
  for (uint64_t i = 0; i < n; ++i) h_ids_.push_back(ids ? ids[i] : base + i);
  dirty_ = true;
}

bool BruteForceIndex::remove(uint64_t id) {
  std::lock_guard<std::mutex> g(mu_);
  const auto it = std::find(h_ids_.begin(), h_ids_.end(), id);
  if (it == h_ids_.end()) return false;
  const uint64_t idx = (uint64_t)(it - h_ids_.begin()), last = h_ids_.size() - 1;
  h_ids_[idx] = h_ids_[last];
  h_ids_.pop_back();
  if (idx != last) std::memcpy(&h_rows_[idx * dim_], &h_rows_[last * dim_], 4 * (size_t)dim_);
  h_rows_.resize(last * dim_);
  dirty_ = true;
  return true;
}

void BruteForceIndex::sync_device() {
  if (!dirty_) return;
  // the rows are replaced on the handle's own stream: the previous call's
  // kernels (on any stream) finish first
  order_.wait_host();
  const uint64_t n = h_ids_.size();
  ld_ = std::max<uint64_t>(256, (n + 255) / 256 * 256);
  if (n) {
    rows_.upload(h_rows_.data(), n * dim_, stream_);
    dataT_.reserve(ld_ * dim_);
    FDB_HIP(launch_transpose_rows(rows_.p, n, (int)dim_, ld_, dataT_.p, stream_));
    row_norm_.reserve(n);
    FDB_HIP(launch_row_norms(rows_.p, n, (int)dim_, row_norm_.p, stream_));
    ids_.upload(h_ids_.data(), n, stream_);
    std::vector<float> rn(n);
    FDB_HIP(hipMemcpyAsync(rn.data(), row_norm_.p, 4 * n, hipMemcpyDeviceToHost, stream_));
    FDB_HIP(hipStreamSynchronize(stream_));
    rnmax_ = 0.0f;
    for (float v : rn) rnmax_ = std::max(rnmax_, v);  // NaN rows leave it unchanged
    h16_.build(rows_.p, row_norm_.p, n, (int)dim_, (int)metric_, stream_);
  } else {
    h16_.ok = false;
  }
  n_dev_ = n;
  dirty_ = false;
}

BruteForceIndex::~BruteForceIndex() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& e : ev_)
    if (e) (void)hipEventDestroy(e);
  if (stream_) (void)hipStreamDestroy(stream_);
}

bool FlatSearcher::screenable(int metric, int dim, uint32_t k) {
  return metric != FDB_METRIC_MANHATTAN && dim % 4 == 0 && dim <= 512 && k > 0 && k + 16 <= 128;
}

// Exact VALU scan.  With flags, only queries flagged nonzero are rewritten
// (the fallback of the screening path).  Query slices of at most 65535 tiles
// (the grid's y limit).  Per slice, row chunks: enough workgroups to fill the
// GPU; the partial lists are capped at 512 MB in all and at 2^20 entries per
// query (one wave merges them).
void FlatSearcher::exact(const FlatRows& x, int metric, const float* d_qs, const float* q_norm,
                         uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists, uint32_t* d_counts,
                         hipStream_t s, const int* flags) {
  const uint64_t n = x.n;
  const uint64_t slice = 65535ull * kQB;
  for (uint64_t q0 = 0; q0 < nq; q0 += slice) {
    const uint64_t m = std::min(slice, nq - q0);
    const uint64_t qtiles = (m + kQB - 1) / kQB;
    uint64_t want = std::max<uint64_t>(1, 4096 / qtiles);
    const uint64_t cap =
        std::max<uint64_t>(1, std::min<uint64_t>((512ull << 20) / (m * k * 8), (1u << 20) / k));
    want = std::min(want, cap);
    uint64_t chunk_rows = (n + want - 1) / want;
    chunk_rows = std::max<uint64_t>(256, (chunk_rows + 255) / 256 * 256);
    const uint32_t nchunks = (uint32_t)((n + chunk_rows - 1) / chunk_rows);
    part_d_.reserve(m * nchunks * k);
    part_k_.reserve(m * nchunks * k);
    FlatTopkArgs a{};
    a.queries = d_qs + q0 * x.dim;
    a.nq = m;
    a.dim = x.dim;
    a.dataT = x.dataT;
    a.ld = x.ld;
    a.n = n;
    a.row_norm = x.row_norm;
    a.q_norm = q_norm ? q_norm + q0 : nullptr;
    a.chunk_rows = chunk_rows;
    a.nchunks = nchunks;
    a.metric = metric;
    a.k = (int)k;
    a.part_d = part_d_.p;
    a.part_key = part_k_.p;
    a.flags = flags ? flags + q0 : nullptr;
    FDB_HIP(launch_flat_topk(a, s));
    FDB_HIP(launch_merge_parts(part_d_.p, part_k_.p, m, nchunks, (int)k, x.ids, d_ids + q0 * k,
                               d_dists + q0 * k, d_counts + q0, s, a.flags));
  }
}

// MFMA screening, exact rescoring of K' candidates, exact scan of the
// queries whose check failed.  Query slices of at most 65536; per slice,
// row chunks for about 2048 workgroups, partial lists capped at 512 MB.
void FlatSearcher::screen(const FlatRows& x, int metric, const float* d_qs, const float* q_norm,
                          uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists, uint32_t* d_counts,
                          hipStream_t s) {
  const uint64_t n = x.n;
  const int kp = (k + 16 <= 64) ? 64 : 128;
  flags_.reserve(nq);
  fallbacks_.reserve(1);
  hipLaunchKernelGGL(clear_u32, dim3(1), dim3(1), 0, s, fallbacks_.p);
  FDB_HIP(hipGetLastError());
  const uint64_t slice = 65536;
  for (uint64_t q0 = 0; q0 < nq; q0 += slice) {
    const uint64_t m = std::min(slice, nq - q0);
    const uint64_t qtiles = (m + kSQ - 1) / kSQ;
    uint64_t want = std::max<uint64_t>(1, 2048 / qtiles);
    want = std::min<uint64_t>(want, std::max<uint64_t>(1, (512ull << 20) / (m * kp * 8)));
    uint64_t chunk_rows = (n + want - 1) / want;
    chunk_rows = std::max<uint64_t>(256, (chunk_rows + 255) / 256 * 256);
    const uint32_t nchunks = (uint32_t)((n + chunk_rows - 1) / chunk_rows);
    part_d_.reserve(m * nchunks * kp);
    part_k_.reserve(m * nchunks * kp);
    cand_d_.reserve(m * kp);
    cand_k_.reserve(m * kp);
    cand_c_.reserve(m);
    ScreenArgs a{};
    a.queries = d_qs + q0 * x.dim;
    a.nq = m;
    a.dim = x.dim;
    a.dataT = x.dataT;
    a.ld = x.ld;
    a.n = n;
    a.row_norm = x.row_norm;
    a.q_norm = q_norm + q0;
    a.chunk_rows = chunk_rows;
    a.nchunks = nchunks;
    a.metric = metric;
    a.kp = kp;
    a.part_d = part_d_.p;
    a.part_key = part_k_.p;
    FDB_HIP(launch_mfma_screen(a, s));
    FDB_HIP(launch_merge_parts(part_d_.p, part_k_.p, m, nchunks, kp, nullptr, cand_k_.p, cand_d_.p,
                               cand_c_.p, s));
    RescoreArgs r{};
    r.queries = a.queries;
    r.dim = x.dim;
    r.rows = x.rows;
    r.row_norm = x.row_norm;
    r.q_norm = a.q_norm;
    r.rnmax = x.rnmax;
    r.cand_keys = cand_k_.p;
    r.cand_d = cand_d_.p;
    r.cand_counts = cand_c_.p;
    r.kp = kp;
    r.metric = metric;
    r.k = (int)k;
    r.ids = x.ids;
    r.out_ids = d_ids + q0 * k;
    r.out_d = d_dists + q0 * k;
    r.out_counts = d_counts + q0;
    r.flags = flags_.p + q0;
    r.fallbacks = fallbacks_.p;
    FDB_HIP(launch_rescore(r, m, s));
  }
  exact(x, metric, d_qs, q_norm, nq, k, d_ids, d_dists, d_counts, s, flags_.p);
}

void CoarseQuantizer::init(const float* centroids, const float* centT, uint32_t nlist, uint32_t dim,
                           hipStream_t s) {
  cent_ = centroids;
  centT_ = centT;
  nlist_ = nlist;
  dim_ = dim;
  c16_.build(centroids, nlist, dim, s);
}

// Screening (fdb_coarse16.hpp) where it applies, then the exact kernel on the
// queries it flagged; else the exact kernel, in parts for batches too small
// to fill the GPU.
void CoarseQuantizer::select(const float* d_qs, uint64_t nq, uint32_t np, int32_t* probes, float* dists,
                             int* err, hipStream_t s) {
  if (nq == 0 || np == 0) return;
  if (mode_ != 1 && nlist_ >= 256 && c16_.serves(np)) {
    flags_.reserve(nq);
    c16_.select(d_qs, nq, np, cent_, probes, dists, flags_.p, s);
    FDB_HIP(launch_coarse_select(d_qs, nq, (int)dim_, centT_, (int)nlist_, (int)np, probes, dists, err, s, nullptr,
                                 nullptr, 0, flags_.p));
    return;
  }
  const uint64_t parts = (uint64_t)coarse_parts(nq, (int)nlist_, (int)np);
  const uint64_t cap = parts > 1 ? nq * parts * np : 0;
  if (cap) {
    part_d_.reserve(cap);
    part_k_.reserve(cap);
  }
  FDB_HIP(launch_coarse_select(d_qs, nq, (int)dim_, centT_, (int)nlist_, (int)np, probes, dists, err, s,
                               part_d_.p, part_k_.p, cap));
}

void CoarseQuantizer::select_one_part(const float* d_qs, uint64_t nq, uint32_t np, int32_t* probes, int* err,
                                      hipStream_t s) const {
  if (nq == 0 || np == 0) return;
  FDB_HIP(launch_coarse_select(d_qs, nq, (int)dim_, centT_, (int)nlist_, (int)np, probes, nullptr, err, s, nullptr,
                               nullptr, 0));
}

// Automatic mode screens when there are at least 2^26 (query, row) pairs;
// below that the launch sequence costs more than the exact scan.
bool BruteForceIndex::screen_applies(uint64_t nq, uint32_t k) const {
  if (!FlatSearcher::screenable((int)metric_, (int)dim_, k) || n_dev_ <= 64 || screen_mode_ == 1)
    return false;
  return screen_mode_ >= 2 || nq * n_dev_ >= (1ull << 26);
}

FlatRows BruteForceIndex::flat_rows() const {
  return FlatRows{dataT_.p, ld_, n_dev_, (int)dim_, rows_.p, row_norm_.p, rnmax_, ids_.p};
}

void BruteForceIndex::run(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                          float* d_dists, uint32_t* d_counts, hipStream_t s) {
  if (nq == 0) return;
  path_ = 0;
  if (k == 0 || n_dev_ == 0) {
    hipLaunchKernelGGL(fill_empty, dim3(nblocks(nq * std::max<uint32_t>(k, 1), 256)), dim3(256), 0, s,
                       nq, k, d_ids, d_dists, d_counts);
    FDB_HIP(hipGetLastError());
    return;
  }
  if (k > 1024) throw Error(FDB_ERR_UNSUPPORTED, "k above 1024");
  const bool screen = screen_applies(nq, k);
  if (metric_ == FDB_METRIC_COSINE || screen) {
    qn_.reserve(nq);
    FDB_HIP(launch_row_norms(d_qs, nq, dim_, qn_.p, s));
  }
  if (screen) {
    if (screen_mode_ != 3 && FlatSearcher::screenable16(h16_, (int)metric_, k)) {
      srch_.screen16(flat_rows(), h16_, (int)metric_, d_qs, qn_.p, nq, k, d_ids, d_dists, d_counts, s);
      path_ = 2;
    } else {
      srch_.screen(flat_rows(), (int)metric_, d_qs, qn_.p, nq, k, d_ids, d_dists, d_counts, s);
      path_ = 1;
    }
  } else {
    srch_.exact(flat_rows(), (int)metric_, d_qs, qn_.p, nq, k, d_ids, d_dists, d_counts, s);
  }
}

uint64_t BruteForceIndex::last_fallbacks(hipStream_t s) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, s ? s : stream_);
  if (path_ == 0 || !srch_.fallbacks()) return 0;  // the last search did not screen
  FDB_HIP(hipStreamSynchronize(s ? s : stream_));
  uint32_t v = 0;
  FDB_HIP(hipMemcpy(&v, srch_.fallbacks(), 4, hipMemcpyDeviceToHost));
  return v;
}

uint32_t BruteForceIndex::search(const float* q, uint32_t k, uint64_t* ids, float* dists) {
  uint32_t c = 0;
  batch_search(q, 1, k, ids, dists, &c);
  return c;
}

void BruteForceIndex::batch_search(const float* qs, uint64_t nq, uint32_t k, uint64_t* ids,
                                   float* dists, uint32_t* counts) {
  if (nq == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  sync_device();
  q_.upload(qs, nq * dim_, stream_);
  const uint32_t kk = std::max<uint32_t>(k, 1);
  out_i_.reserve(nq * kk);
  out_d_.reserve(nq * kk);
  out_c_.reserve(nq);
  run(q_.p, nq, k, out_i_.p, out_d_.p, out_c_.p, stream_);
  if (k) {
    FDB_HIP(hipMemcpyAsync(ids, out_i_.p, 8 * nq * k, hipMemcpyDeviceToHost, stream_));
    FDB_HIP(hipMemcpyAsync(dists, out_d_.p, 4 * nq * k, hipMemcpyDeviceToHost, stream_));
  }
  FDB_HIP(hipMemcpyAsync(counts, out_c_.p, 4 * nq, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
}

void BruteForceIndex::batch_search_device(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                                          float* d_dists, uint32_t* d_counts, hipStream_t s,
                                          float* ms) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, s ? s : stream_);
  sync_device();
  hipStream_t st = s ? s : stream_;
  if (ms) FDB_HIP(hipEventRecord(ev_[0], st));
  run(d_qs, nq, k, d_ids, d_dists, d_counts, st);
  if (ms) {
    FDB_HIP(hipEventRecord(ev_[1], st));
    FDB_HIP(hipEventSynchronize(ev_[1]));
    FDB_HIP(hipEventElapsedTime(ms, ev_[0], ev_[1]));
  }
}

// ===========================================================================
// IVFIndex
// ===========================================================================
IvfFlatIndex::IvfFlatIndex(const float* centroids, uint32_t nlist, uint32_t dim, const uint64_t* offsets,
                           const uint64_t* ids, const float* rows, uint32_t metric)
    : nlist_(nlist), dim_(dim), metric_(metric) {
  if (nlist == 0 || dim == 0) throw Error(FDB_ERR_INVALID_ARGUMENT, "nlist and dim must be positive");
  if (dim > 2048) throw Error(FDB_ERR_UNSUPPORTED, "dim above 2048");
  if (metric > 4) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown metric");
  h_centroids_.assign(centroids, centroids + (size_t)nlist * dim);
  h_offsets_.assign(offsets, offsets + nlist + 1);
  if (h_offsets_[0] != 0) throw Error(FDB_ERR_INVALID_ARGUMENT, "offsets must start at 0");
  for (uint32_t l = 0; l < nlist; ++l)
    if (h_offsets_[l + 1] < h_offsets_[l]) throw Error(FDB_ERR_INVALID_ARGUMENT, "offsets decrease");
  const uint64_t n = h_offsets_[nlist];
  if (n >= 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "more than 2^32-2 rows");
  if (n && (!ids || !rows)) throw Error(FDB_ERR_INVALID_ARGUMENT, "null ids or rows");
  h_ids_.assign(ids, ids + n);
  h_rows_.assign(rows, rows + n * dim);
  FDB_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  for (auto& e : ev_) FDB_HIP(hipEventCreate(&e));
  // centroids for the coarse kernel
  cent_.upload(h_centroids_.data(), h_centroids_.size(), stream_);
  centT_.reserve((size_t)centT_ld(nlist) * dim);
  FDB_HIP(launch_transpose_centroids(cent_.p, nlist, dim, centT_.p, stream_));
  coarse_.init(cent_.p, centT_.p, nlist, dim, stream_);
  // list blocks [dim][lld_p], lld_p = len_p rounded up to 4
  std::vector<uint64_t> boff(nlist);
  uint64_t tot = 0;
  for (uint32_t l = 0; l < nlist; ++l) {
    boff[l] = tot;
    tot += (h_offsets_[l + 1] - h_offsets_[l] + 3) / 4 * 4 * (uint64_t)dim;
  }
  data_.reserve(std::max<uint64_t>(tot, 4));
  rowsl_.upload(h_rows_.data(), std::max<uint64_t>(n * dim, 1), stream_);
  for (uint32_t l = 0; l < nlist; ++l) {
    const uint64_t s = h_offsets_[l], len = h_offsets_[l + 1] - s;
    if (len == 0) continue;
    FDB_HIP(launch_transpose_rows(rowsl_.p + s * dim, len, dim, (len + 3) / 4 * 4, data_.p + boff[l], stream_));
  }
  if (metric == FDB_METRIC_COSINE) {
    row_norm_.reserve(std::max<uint64_t>(n, 1));
    FDB_HIP(launch_row_norms(rowsl_.p, n, dim, row_norm_.p, stream_));
  }
  FDB_HIP(hipStreamSynchronize(stream_));
  boff_.upload(boff.data(), nlist, stream_);
  std::vector<uint32_t> ro(h_offsets_.begin(), h_offsets_.end());
  row_off_.upload(ro.data(), ro.size(), stream_);
  if (metric == FDB_METRIC_EUCLIDEAN || metric == FDB_METRIC_EUCLIDEAN_SQUARED || metric == FDB_METRIC_MANHATTAN)
    l16_.build(rowsl_.p, h_offsets_, nlist, (int)dim, row_off_.p, stream_);
  ids_.upload(h_ids_.data(), std::max<uint64_t>(n, 1), stream_);
  err_.reserve(1);
  hipLaunchKernelGGL(clear_flag, dim3(1), dim3(1), 0, stream_, err_.p);
  FDB_HIP(hipGetLastError());
  FDB_HIP(hipStreamSynchronize(stream_));
}

IvfFlatIndex::~IvfFlatIndex() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& e : ev_)
    if (e) (void)hipEventDestroy(e);
  if (stream_) (void)hipStreamDestroy(stream_);
}

// IVFIndex::build, ivf.rs:91-119: k-means (DEFAULT_MAX_ITERATIONS = 100,
// constants.rs:32) over every vector, then first-minimum assignment with the
// vectors kept in input order inside each list.  The k-means initialisation
// draws from splitmix64_at(seed, 1).
IvfFlatIndex* IvfFlatIndex::build(const float* vectors, const uint64_t* ids, uint64_t n, uint32_t dim,
                                  uint32_t nlist, uint32_t metric, uint32_t max_iters, uint64_t seed) {
  if (n == 0 || dim == 0 || nlist == 0) throw Error(FDB_ERR_INVALID_ARGUMENT, "n, dim, nlist must be positive");
  if (dim > 2048) throw Error(FDB_ERR_UNSUPPORTED, "dim above 2048");
  if (n >= 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "more than 2^32-2 vectors");
  for (uint64_t i = 0; i < n * dim; ++i)
    if (std::isnan(vectors[i])) throw Error(FDB_ERR_NAN, "NaN in the vectors to index");
  hipStream_t s;
  FDB_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  struct G {
    hipStream_t s;
    ~G() {
      (void)hipStreamSynchronize(s);
      (void)hipStreamDestroy(s);
    }
  } guard{s};
  std::vector<float> cents = kmeans_gpu(vectors, n, (int)dim, (int)nlist, (int)max_iters, splitmix64_at(seed, 1), s);
  DevBuf<float> d_vec, d_c, d_cT;
  DevBuf<int32_t> d_a;
  d_vec.upload(vectors, n * dim, s);
  d_c.upload(cents.data(), cents.size(), s);
  d_cT.reserve((size_t)centT_ld(nlist) * dim);
  d_a.reserve(n);
  FDB_HIP(launch_transpose_centroids(d_c.p, nlist, dim, d_cT.p, s));
  FDB_HIP(launch_assign(d_vec.p, n, dim, d_cT.p, nlist, d_a.p, s));
  std::vector<int32_t> assign(n);
  FDB_HIP(hipMemcpyAsync(assign.data(), d_a.p, 4 * n, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  std::vector<uint64_t> off(nlist + 1, 0);
  for (int32_t a : assign) {
    if (a < 0 || a >= (int32_t)nlist) throw Error(FDB_ERR_NAN, "assignment failed (NaN distance)");
    off[a + 1]++;
  }
  for (uint32_t l = 0; l < nlist; ++l) off[l + 1] += off[l];
  std::vector<uint64_t> fill(off.begin(), off.end() - 1), lids(n);
  std::vector<float> rows(n * dim);
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t p = fill[assign[i]]++;
    lids[p] = ids ? ids[i] : i;
    std::memcpy(&rows[p * dim], vectors + i * dim, 4 * dim);
  }
  return new IvfFlatIndex(cents.data(), nlist, dim, off.data(), lids.data(), rows.data(), metric);
}

void IvfFlatIndex::export_to(float* centroids, uint64_t* offsets, uint64_t* ids, float* rows) const {
  if (centroids) std::memcpy(centroids, h_centroids_.data(), 4 * h_centroids_.size());
  if (offsets) std::memcpy(offsets, h_offsets_.data(), 8 * h_offsets_.size());
  if (ids) std::memcpy(ids, h_ids_.data(), 8 * h_ids_.size());
  if (rows) std::memcpy(rows, h_rows_.data(), 4 * h_rows_.size());
}

void IvfFlatIndex::run(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists,
                       uint32_t* d_counts, hipStream_t s, float* coarse_ms, float* scan_ms) {
  if (nq == 0) return;
  uint32_t np = (uint32_t)std::min<uint64_t>(nprobe(), nlist_);  // take(nprobe): 0 lists when 0
  if (k == 0 || np == 0) {
    hipLaunchKernelGGL(fill_empty, dim3(nblocks(nq * std::max<uint32_t>(k, 1), 256)), dim3(256), 0, s,
                       nq, k, d_ids, d_dists, d_counts);
    FDB_HIP(hipGetLastError());
    if (coarse_ms) *coarse_ms = 0.0f;
    if (scan_ms) *scan_ms = 0.0f;
    return;
  }
  if (k > 1024) throw Error(FDB_ERR_UNSUPPORTED, "k above 1024");
  if (np > 1024 && np < nlist_) throw Error(FDB_ERR_UNSUPPORTED, "nprobe above 1024");
  const bool timed = coarse_ms || scan_ms;
  probes_.reserve(nq * np);
  if (timed) FDB_HIP(hipEventRecord(ev_[0], s));
  if (np >= nlist_) {
    np = nlist_;
    hipLaunchKernelGGL(iota_probes, dim3(nblocks(nq * np, 256)), dim3(256), 0, s, nq, np, probes_.p);
    FDB_HIP(hipGetLastError());
  } else {
    coarse_.select(d_qs, nq, np, probes_.p, nullptr, err_.p, s);
  }
  if (timed) FDB_HIP(hipEventRecord(ev_[1], s));
  const bool l1 = metric_ == FDB_METRIC_MANHATTAN;
  const bool l2 = metric_ == FDB_METRIC_EUCLIDEAN || metric_ == FDB_METRIC_EUCLIDEAN_SQUARED;
  // the exact scan of queries [q0, q0 + m), those flagged only when flags
  auto exact_scan = [&](uint64_t q0, uint64_t m, const int* flags) {
    IvfFlatScanArgs a{};
    a.queries = d_qs + q0 * dim_;
    a.nq = m;
    a.dim = (int)dim_;
    a.probes = probes_.p + q0 * np;
    a.np = (int)np;
    a.nlist = (int)nlist_;
    a.data = data_.p;
    a.boff = boff_.p;
    a.row_off = row_off_.p;
    a.row_norm = row_norm_.p;
    a.q_norm = qn_.p ? qn_.p + q0 : nullptr;
    a.ids = ids_.p;
    a.metric = (int)metric_;
    a.k = (int)k;
    a.out_ids = d_ids + q0 * k;
    a.out_d = d_dists + q0 * k;
    a.out_counts = d_counts + q0;
    a.flags = flags;
    FDB_HIP(launch_ivf_flat_scan(a, s));
  };
  // list screening on the matrix cores (fdb_ivfpq16.hpp over the rows):
  // pairs grouped by list, each list's blocks multiplied against up to 256
  // queries at a time
  const uint64_t scanned = nlist_ ? h_ids_.size() * np / nlist_ : 0;
  bool lists = search_mode_ != 1 && l2 && np >= 2 && dim_ <= 256 && nlist_ <= 8192 &&
               (search_mode_ == 2 || nq * scanned >= kListScreenMinWork);
  if (lists && !p16_tried_) {
    p16_.build_rows(rowsl_.p, row_off_.p, h_offsets_, nlist_, (int)dim_, s);
    p16_tried_ = true;
  }
  lists = lists && p16_.ok;
  // (the exact rescoring reads rows as float4: dim a multiple of 4, <= 512)
  const bool screen = !lists && search_mode_ != 1 && l16_.ok && k + 16 <= 128 && dim_ % 4 == 0 && dim_ <= 512 &&
                      (l1 || l2);
  if (metric_ == FDB_METRIC_COSINE || screen) {
    qn_.reserve(nq);
    FDB_HIP(launch_row_norms(d_qs, nq, dim_, qn_.p, s));
  }
  path_ = 0;
  if (timed) screen_kernel_ms_ = 0.0f;
  if (lists) {
    // each slice screened and rescored, then its flagged queries scanned
    // exactly
    p16s_.reset_stats(s);
    p16s_.set_timing(timed);
    const uint64_t sl = std::min<uint64_t>(nq, Pq16Searcher::slice((int)k));
    for (uint64_t q0 = 0; q0 < nq; q0 += sl) {
      const uint64_t m = std::min<uint64_t>(sl, nq - q0);
      Pq16SearchArgs sa{};
      sa.queries = d_qs + q0 * dim_;
      sa.nq = m;
      sa.probes = probes_.p + q0 * np;
      sa.np = (int)np;
      sa.centroids = cent_.p;
      sa.ids = ids_.p;
      sa.list_off = row_off_.p;
      sa.k = (int)k;
      sa.order = 0;
      sa.rows = rowsl_.p;
      sa.sqrt_out = metric_ == FDB_METRIC_EUCLIDEAN ? 1 : 0;
      sa.out_ids = d_ids + q0 * k;
      sa.out_d = d_dists + q0 * k;
      sa.out_counts = d_counts + q0;
      p16s_.search(p16_, sa, s);
      exact_scan(q0, m, p16s_.flags());
    }
    if (timed) screen_kernel_ms_ = p16s_.screen_ms();
    p16s_.set_timing(false);
    path_ = 3;
  } else {
    if (screen) {
      // fp16 screening of the probed lists, exact rescoring of K' candidates,
      // then the exact scan for the queries the bound does not settle
      const int kp = (k + 16 <= 64) ? 64 : 128;
      cand_d_.reserve(nq * kp);
      cand_k_.reserve(nq * kp);
      cand_c_.reserve(nq);
      abound_.reserve(nq);
      flags_.reserve(nq);
      fallbacks_.reserve(1);
      hipLaunchKernelGGL(clear_u32, dim3(1), dim3(1), 0, s, fallbacks_.p);
      FDB_HIP(hipGetLastError());
      FDB_HIP(l16_.screen(d_qs, nq, probes_.p, np, nlist_, row_off_.p, l1, kp, cand_d_.p, cand_k_.p, cand_c_.p,
                          abound_.p, s));
      RescoreArgs r{};
      r.queries = d_qs;
      r.dim = (int)dim_;
      r.rows = rowsl_.p;
      r.row_norm = row_norm_.p;
      r.q_norm = qn_.p;
      r.cand_keys = cand_k_.p;
      r.cand_d = cand_d_.p;
      r.cand_counts = cand_c_.p;
      r.kp = kp;
      r.metric = (int)metric_;
      r.k = (int)k;
      r.ids = ids_.p;
      r.out_ids = d_ids;
      r.out_d = d_dists;
      r.out_counts = d_counts;
      r.flags = flags_.p;
      r.fallbacks = fallbacks_.p;
      r.abound = abound_.p;
      r.bkind = kBoundIvf16;
      r.n = h_ids_.size();
      r.xmag = l1 ? l16_.xnorm1_max : l16_.xnorm2_max;
      r.xexp = l16_.xexp;
      FDB_HIP(launch_rescore(r, nq, s));
      path_ = 2;
    }
    exact_scan(0, nq, screen ? flags_.p : nullptr);
  }
  if (timed) {
    FDB_HIP(hipEventRecord(ev_[2], s));
    FDB_HIP(hipEventSynchronize(ev_[2]));
    if (coarse_ms) FDB_HIP(hipEventElapsedTime(coarse_ms, ev_[0], ev_[1]));
    if (scan_ms) FDB_HIP(hipEventElapsedTime(scan_ms, ev_[1], ev_[2]));
  }
}

uint64_t IvfFlatIndex::last_fallbacks(hipStream_t s) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, s ? s : stream_);
  if (path_ == 3) {
    uint64_t fb = 0, cand = 0;
    p16s_.read_stats(fb, cand, s ? s : stream_);
    return fb;
  }
  if (path_ == 0 || !fallbacks_.p) return 0;  // the last search did not screen
  FDB_HIP(hipStreamSynchronize(s ? s : stream_));
  uint32_t v = 0;
  FDB_HIP(hipMemcpy(&v, fallbacks_.p, 4, hipMemcpyDeviceToHost));
  return v;
}

void IvfFlatIndex::probe(const float* qs, uint64_t nq, uint32_t nprobe, int32_t* lists) {
  if (nq == 0 || nprobe == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  if (nprobe > nlist_) throw Error(FDB_ERR_INVALID_ARGUMENT, "nprobe above nlist");
  if (nprobe > 1024) throw Error(FDB_ERR_UNSUPPORTED, "nprobe above 1024");
  q_.upload(qs, nq * dim_, stream_);
  probes_.reserve(nq * nprobe);
  coarse_.select(q_.p, nq, nprobe, probes_.p, nullptr, err_.p, stream_);
  FDB_HIP(hipMemcpyAsync(lists, probes_.p, 4 * nq * nprobe, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
}

bool IvfFlatIndex::sync(hipStream_t s) {
  std::lock_guard<std::mutex> g(mu_);
  FDB_HIP(hipStreamSynchronize(s ? s : stream_));
  int flag = 0;
  FDB_HIP(hipMemcpy(&flag, err_.p, 4, hipMemcpyDeviceToHost));
  if (flag) {
    hipLaunchKernelGGL(clear_flag, dim3(1), dim3(1), 0, stream_, err_.p);
    FDB_HIP(hipGetLastError());
    FDB_HIP(hipStreamSynchronize(stream_));
  }
  return flag != 0;
}

void IvfFlatIndex::batch_search(const float* qs, uint64_t nq, uint32_t k, uint64_t* ids, float* dists,
                                uint32_t* counts) {
  if (nq == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  q_.upload(qs, nq * dim_, stream_);
  const uint32_t kk = std::max<uint32_t>(k, 1);
  out_i_.reserve(nq * kk);
  out_d_.reserve(nq * kk);
  out_c_.reserve(nq);
  run(q_.p, nq, k, out_i_.p, out_d_.p, out_c_.p, stream_, nullptr, nullptr);
  if (k) {
    FDB_HIP(hipMemcpyAsync(ids, out_i_.p, 8 * nq * k, hipMemcpyDeviceToHost, stream_));
    FDB_HIP(hipMemcpyAsync(dists, out_d_.p, 4 * nq * k, hipMemcpyDeviceToHost, stream_));
  }
  FDB_HIP(hipMemcpyAsync(counts, out_c_.p, 4 * nq, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
  int flag = 0;
  FDB_HIP(hipMemcpy(&flag, err_.p, 4, hipMemcpyDeviceToHost));
  if (flag) {
    hipLaunchKernelGGL(clear_flag, dim3(1), dim3(1), 0, stream_, err_.p);
    FDB_HIP(hipStreamSynchronize(stream_));
    throw Error(FDB_ERR_NAN, "NaN centroid distance (a query contains NaN)");
  }
}

void IvfFlatIndex::batch_search_device(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                                       float* d_dists, uint32_t* d_counts, hipStream_t s,
                                       float* coarse_ms, float* scan_ms) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, s ? s : stream_);
  run(d_qs, nq, k, d_ids, d_dists, d_counts, s ? s : stream_, coarse_ms, scan_ms);
}

}  // namespace fdb
