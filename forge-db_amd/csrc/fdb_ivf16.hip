// IVF (full vectors) screening on fp16 copies of the lists, followed by the
// exact rescoring of fdb_flat.hip.  The reference scans every vector of the
// probed lists with metric.compute (ivf.rs:179-216, :292-297); here the scan
// reads half-precision rows to pick K' candidates per query, their distances
// are recomputed exactly in the reference's order, and ivf16_bound shows
// that no other scanned row can enter the top k (queries it cannot settle
// are rescanned exactly).  Euclidean, squared Euclidean and Manhattan.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "fdb_device.hpp"
#include "fdb_flat.hpp"

namespace fdb {

namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int kT = 256;

__device__ __forceinline__ uint32_t fbits(float v) { return __float_as_uint(v); }

__global__ void init_ivf_stats(uint32_t* s) {
  for (int i = 0; i < 4; ++i) s[i] = 0;
}

// stats: [0] bits of max |x_i| (non-finite values compare above every finite
// one), [1] bits of max sum x_i^2, [2] bits of max sum |x_i| (each row's sums
// in fp32, any order; the caller widens them).  Grid-stride, one wave per row.
__global__ __launch_bounds__(kT) void ivf_rows_stats_kernel(const float* __restrict__ rows, uint64_t n, int dim,
                                                            uint32_t* __restrict__ stats) {
  __shared__ uint32_t red[3][4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t mabs = 0, mn2 = 0, mn1 = 0;
  for (uint64_t r = (uint64_t)blockIdx.x * 4 + wave; r < n; r += (uint64_t)gridDim.x * 4) {
    float s2 = 0.0f, s1 = 0.0f;
    uint32_t ma = 0;
    for (int d = lane; d < dim; d += 64) {
      const float v = rows[r * dim + d];
      s2 = __builtin_fmaf(v, v, s2);
      s1 += __builtin_fabsf(v);
      ma = std::max(ma, fbits(v) & 0x7FFFFFFFu);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      s2 += __shfl_xor(s2, off);
      s1 += __shfl_xor(s1, off);
      ma = std::max(ma, (uint32_t)__shfl_xor((int)ma, off));
    }
    mabs = std::max(mabs, ma);
    mn2 = std::max(mn2, fbits(s2) & 0x7FFFFFFFu);
    mn1 = std::max(mn1, fbits(s1) & 0x7FFFFFFFu);
  }
  if (lane == 0) {
    red[0][wave] = mabs;
    red[1][wave] = mn2;
    red[2][wave] = mn1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w)
      for (int i = 0; i < 3; ++i) red[i][0] = std::max(red[i][0], red[i][w]);
    for (int i = 0; i < 3; ++i) atomicMax(&stats[i], red[i][0]);
  }
}

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  h2 v;
  v.x = (_Float16)a;
  v.y = (_Float16)b;
  return __builtin_bit_cast(uint32_t, v);
}

__global__ void fill_u32(uint32_t* p, uint64_t n) {
  const uint64_t i = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (i < n) p[i] = 0;
}

// List blocks of dimension pairs: list p holds [dim2][lld_p] words, lld_p =
// |L_p| rounded up to 4, word (j, r) = the pair (x_{2j}, x_{2j+1}) * 2^e of
// its row r as two halves, so a lane reads 4 rows of a pair as one 16-byte
// load.  One thread per (row, pair); rows in list order.
__global__ __launch_bounds__(kT) void ivf_rows_to_h16_kernel(const float* __restrict__ rows, uint64_t n, int dim,
                                                             int dim2, const uint32_t* __restrict__ row_list,
                                                             const uint32_t* __restrict__ row_off,
                                                             const uint64_t* __restrict__ boff, int ex,
                                                             uint32_t* __restrict__ out) {
  const uint64_t t = (uint64_t)blockIdx.x * kT + threadIdx.x;
  if (t >= n * (uint64_t)dim2) return;
  const uint64_t r = t / (uint64_t)dim2;
  const int j = (int)(t - r * (uint64_t)dim2);
  const uint32_t p = row_list[r];
  const uint32_t s = row_off[p];
  const uint64_t lld = ((uint64_t)(row_off[p + 1] - s) + 3) / 4 * 4;
  const float a = ldexpf(rows[r * dim + 2 * j], ex);
  const float b = 2 * j + 1 < dim ? ldexpf(rows[r * dim + 2 * j + 1], ex) : 0.0f;
  out[boff[p] + (uint64_t)j * lld + (r - s)] = pack_h2(a, b);
}

struct Ivf16Args {
  const float* queries;  // [nq][dim]
  uint64_t nq;
  int dim, dim2;
  const int32_t* probes;  // [nq][np]
  int np, nlist;
  const uint32_t* data;   // list blocks of half pairs
  const uint64_t* boff;   // [nlist] word offset of each block
  const uint32_t* row_off;  // [nlist+1]
  int xexp;
  int kp;
  float* cand_d;       // [nq][kp]
  uint64_t* cand_k;    // [nq][kp] list positions
  uint32_t* cand_c;    // [nq]
  float* abound;       // [nq]
};

// One workgroup (4 waves) per query; probed list j goes to wave j % 4.  The
// query's scaled half pairs sit in LDS (a wave-uniform broadcast per pair);
// each lane takes 4 adjacent rows and accumulates per pair
//   L2: dot2(d, d) of the packed difference d = q - x (rounded to fp16);
//   L1: dot2(|d|, 1).
// Every scanned row is offered (value, list position) to the wave's K' list
// through its candidate queue; the 4 lists are merged.  A query whose scaled
// components would leave fp16's range is marked kForceExact.
template <bool L1, int RS>
__global__ __launch_bounds__(kT) void ivf16_screen_kernel(Ivf16Args a) {
  extern __shared__ uint32_t sm[];
  uint32_t* qh = sm;                                           // [dim2]
  uint2* queue = reinterpret_cast<uint2*>(sm + ((a.dim2 + 1) & ~1));  // [4][64]
  __shared__ uint32_t s_bad;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t q = blockIdx.x;
  const int dim = a.dim;
  const float* __restrict__ qv = a.queries + q * (uint64_t)dim;
  if (tid == 0) s_bad = 0;
  __syncthreads();
  // the largest scaled component must stay below 2^14 (then |q - x| < 2^15)
  bool bad = false;
  for (int d = tid; d < dim; d += kT) {
    const float v = ldexpf(__builtin_fabsf(qv[d]), a.xexp);
    bad = bad || !(v < 16384.0f);
  }
  if (__ballot(bad) != 0 && lane == 0) atomicOr(&s_bad, 1u);
  for (int j = tid; j < a.dim2; j += kT)
    qh[j] = pack_h2(ldexpf(qv[2 * j], a.xexp), 2 * j + 1 < dim ? ldexpf(qv[2 * j + 1], a.xexp) : 0.0f);
  __syncthreads();
  const int kp = a.kp;
  if (s_bad) {
    if (tid == 0) {
      a.cand_c[q] = kForceExact;
      a.abound[q] = f_inf();
    }
    return;
  }
  const float unscale = ldexpf(1.0f, L1 ? -a.xexp : -2 * a.xexp);
  WaveTopK<RS> tk;
  tk.init(kp);
  uint2* wq = queue + wave * 64;
  int qn = 0;
  const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
  const int32_t* __restrict__ pr = a.probes + q * (uint64_t)a.np;
  for (int j = wave; j < a.np; j += 4) {
    const int p = pr[j];
    if (p < 0 || p >= a.nlist) continue;  // wave-uniform
    const uint32_t rs = a.row_off[p];
    const uint32_t len = a.row_off[p + 1] - rs;
    const uint64_t lld = ((uint64_t)len + 3) / 4 * 4;
    const uint32_t* __restrict__ blk = a.data + a.boff[p];
    for (uint32_t base = 0; base < len; base += 256) {
      uint64_t c = base + 4 * (uint64_t)lane;
      const bool any = c < len;
      if (!any) c = 0;  // re-read the first rows; nothing is offered
      float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int j2 = 0; j2 < a.dim2; ++j2) {
        const uint4 v = *reinterpret_cast<const uint4*>(blk + (uint64_t)j2 * lld + c);
        const h2 qq = __builtin_bit_cast(h2, qh[j2]);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const h2 d = qq - __builtin_bit_cast(h2, w[u]);
          if constexpr (L1) {
            const h2 ad = __builtin_bit_cast(h2, __builtin_bit_cast(uint32_t, d) & 0x7FFF7FFFu);
            acc[u] = __builtin_amdgcn_fdot2(ad, ones, acc[u], false);
          } else {
            acc[u] = __builtin_amdgcn_fdot2(d, d, acc[u], false);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool in = any && c + u < len;
        tk.offer_queued(acc[u] * unscale, rs + (uint32_t)(c + u), in, wq, qn);
      }
    }
  }
  tk.flush(wq, qn);
  // merge the 4 wave lists in wave 0 (LDS after the query pairs is free)
  __syncthreads();
  float* md = reinterpret_cast<float*>(queue);
  uint32_t* mk = reinterpret_cast<uint32_t*>(md + 4 * 64 * RS);
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    md[wave * 64 * RS + r * 64 + lane] = tk.d[r];
    mk[wave * 64 * RS + r * 64 + lane] = tk.p[r];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < 4; ++w)
#pragma unroll
    for (int r = 0; r < RS; ++r) tk.offer(md[w * 64 * RS + r * 64 + lane], mk[w * 64 * RS + r * 64 + lane]);
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < RS; ++r) {
    const int s = r * 64 + lane;
    const bool valid = tk.p[r] != kNoPos;
    count += (uint32_t)__popcll(__ballot(valid));
    a.cand_d[q * kp + s] = tk.d[r];
    a.cand_k[q * kp + s] = valid ? (uint64_t)tk.p[r] : ~0ull;
  }
  if (lane == 0) {
    a.cand_c[q] = count;
    // every scanned row outside the list screens at or above the K'-th
    a.abound[q] = count >= (uint32_t)kp ? tk.tau : f_inf();
  }
}

unsigned cdiv(uint64_t a, uint64_t b) { return (unsigned)((a + b - 1) / b); }

}  // namespace

void Ivf16Lists::build(const float* d_rows, const std::vector<uint64_t>& offsets, uint32_t nlist, int dim,
                       const uint32_t* d_row_off, hipStream_t s) {
  ok = false;
  const uint64_t n = offsets[nlist];
  dim_ = dim;
  dim2 = (dim + 1) / 2;
  if (n == 0) return;
  stats_.reserve(4);
  hipLaunchKernelGGL(init_ivf_stats, dim3(1), dim3(1), 0, s, stats_.p);
  FDB_HIP(hipGetLastError());
  hipLaunchKernelGGL(ivf_rows_stats_kernel, dim3(std::min<unsigned>(2048, cdiv(n, 4))), dim3(kT), 0, s, d_rows, n,
                     dim, stats_.p);
  FDB_HIP(hipGetLastError());
  uint32_t st[4];
  FDB_HIP(hipMemcpyAsync(st, stats_.p, sizeof(st), hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  float maxabs, n2, n1;
  std::memcpy(&maxabs, &st[0], 4);
  std::memcpy(&n2, &st[1], 4);
  std::memcpy(&n1, &st[2], 4);
  if (!std::isfinite(maxabs) || !std::isfinite(n2) || !std::isfinite(n1)) return;
  int e = 0;
  if (maxabs > 0.0f) {
    int ee;
    (void)std::frexp(maxabs, &ee);
    e = 13 - ee;  // maxabs * 2^e in [2^12, 2^13): differences stay below 2^14
  }
  if (e > 100 || e < -100) return;
  xexp = e;
  // the sums were taken in fp32 in some order: widen them
  const float widen = 1.0f + 2.0f * (float)dim * 5.9604645e-8f;
  xnorm2_max = std::sqrt(n2 * widen) * (1.0f + 1.2e-7f);
  xnorm1_max = n1 * widen;
  std::vector<uint64_t> boff(nlist);
  uint64_t tot = 0;
  std::vector<uint32_t> row_list(n);
  for (uint32_t l = 0; l < nlist; ++l) {
    boff[l] = tot;
    const uint64_t len = offsets[l + 1] - offsets[l];
    tot += (len + 3) / 4 * 4 * (uint64_t)dim2;
    for (uint64_t r = offsets[l]; r < offsets[l + 1]; ++r) row_list[r] = l;
  }
  data_.reserve(std::max<uint64_t>(tot, 4));
  hipLaunchKernelGGL(fill_u32, dim3(cdiv(std::max<uint64_t>(tot, 4), kT)), dim3(kT), 0, s, data_.p,
                     std::max<uint64_t>(tot, 4));
  FDB_HIP(hipGetLastError());
  boff_.upload(boff.data(), nlist, s);
  DevBuf<uint32_t> d_list;
  d_list.upload(row_list.data(), n, s);
  hipLaunchKernelGGL(ivf_rows_to_h16_kernel, dim3(cdiv(n * (uint64_t)dim2, kT)), dim3(kT), 0, s, d_rows, n, dim,
                     dim2, d_list.p, d_row_off, boff_.p, e, data_.p);
  FDB_HIP(hipGetLastError());
  FDB_HIP(hipStreamSynchronize(s));
  ok = true;
}

hipError_t Ivf16Lists::screen(const float* d_qs, uint64_t nq, const int32_t* probes, uint32_t np, uint32_t nlist,
                              const uint32_t* d_row_off, bool l1, int kp, float* cand_d, uint64_t* cand_k,
                              uint32_t* cand_c, float* abound, hipStream_t s) const {
  if (nq == 0) return hipSuccess;
  if (!ok || (kp != 64 && kp != 128)) return hipErrorInvalidValue;
  Ivf16Args a{};
  a.queries = d_qs;
  a.nq = nq;
  a.dim = dim_;
  a.dim2 = dim2;
  a.probes = probes;
  a.np = (int)np;
  a.nlist = (int)nlist;
  a.data = data_.p;
  a.boff = boff_.p;
  a.row_off = d_row_off;
  a.xexp = xexp;
  a.kp = kp;
  a.cand_d = cand_d;
  a.cand_k = cand_k;
  a.cand_c = cand_c;
  a.abound = abound;
  const int RS = kp / 64;
  // query pairs, then the 4 wave queues (later the merge buffer)
  const size_t lds = 4 * (size_t)((dim2 + 1) & ~1) + std::max<size_t>(4 * 64 * 8, 4 * 64 * RS * 8);
  void* fn = l1 ? (RS == 1 ? (void*)ivf16_screen_kernel<true, 1> : (void*)ivf16_screen_kernel<true, 2>)
                : (RS == 1 ? (void*)ivf16_screen_kernel<false, 1> : (void*)ivf16_screen_kernel<false, 2>);
  void* args[] = {(void*)&a};
  return hipLaunchKernel(fn, dim3((unsigned)nq), dim3(kT), args, lds, s);
}

}  // namespace fdb
