// Brute-force screening on the fp16 matrix cores (v_mfma_f32_32x32x16_f16)
// with a ladder of thresholds, followed by the exact rescoring of
// fdb_flat.hip.  The reference computes every distance exactly
// (brute_force.rs:141-146 / :162-225); here the fp16 product only decides
// which rows are rescored, and screen16_eps bounds how far its value can be
// from the reference's, so the results are the reference's (queries the
// bound cannot settle are rescanned exactly).
//
// Stages.  Every stage runs the same kernel over a set of 32-row blocks: a
// row whose screening value is at most the query's threshold tau is
// appended to the query's buffers.  The first stage takes at most 32 evenly
// spaced blocks with tau = +inf; after each stage tau becomes the m-th
// smallest value appended, m chosen so that about 256 rows of the next
// (32x, last 8x larger) sample pass it.  The last stage covers every block;
// the K' smallest of its appends are rescored, and every other row screens
// above min(K'-th value, tau).  The thresholds only steer the amount of
// work: correctness rests on the last stage and the bound.
#include <algorithm>
#include <cmath>
#include <cstring>

#include "fdb_device.hpp"
#include "fdb_flat.hpp"

namespace fdb {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kT16 = 256;          // threads per screening workgroup (4 waves)
constexpr int kStageKiB = 32;      // LDS per workgroup: one stage of row blocks
constexpr uint32_t kSub = 64;      // entries of one append buffer
constexpr uint64_t kSlice = 16384;  // queries per pass
constexpr uint64_t kSubBudget = 1ull << 26;  // append entries per pass (512 MB)

// Exponent e with maxabs * 2^e in [2^13, 2^14); 0 for 0 or non-finite.
__device__ __forceinline__ int scale_exp(float maxabs) {
  if (!(maxabs > 0.0f) || !(maxabs < __builtin_huge_valf())) return 0;
  int e;
  (void)frexpf(maxabs, &e);  // maxabs in [2^(e-1), 2^e)
  return 14 - e;
}

__device__ __forceinline__ uint32_t f2u_abs(float v) { return __float_as_uint(v) & 0x7FFFFFFFu; }

// ---- rows (at index sync) ------------------------------------------------

__global__ void init_stats(uint32_t* s) {
  s[0] = 0;
  s[1] = 0;
  s[2] = 0x7F7FFFFFu;  // FLT_MAX
}

// stats[0]: bits of max |x| (of x / |x| for cosine; NaN/inf compare above
// every finite value); cosine only: stats[1] rows whose squared norm is not
// a finite normal float (zero rows included), stats[2] bits of the smallest
// squared norm.
// Grid-stride over rows, one wave per row at a time; one set of atomics per
// workgroup.
__global__ __launch_bounds__(256) void rows_absmax_kernel(const float* __restrict__ rows, uint64_t n, int dim,
                                                          const float* __restrict__ rn, int cosine,
                                                          uint32_t* __restrict__ stats) {
  __shared__ uint32_t red[3][4];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  uint32_t m = 0, bad = 0, mn = 0x7F7FFFFFu;
  for (uint64_t r = (uint64_t)blockIdx.x * 4 + wave; r < n; r += (uint64_t)gridDim.x * 4) {
    float scale = 1.0f;
    if (cosine) {
      const float nr = rn[r];
      const float inv = 1.0f / __builtin_sqrtf(nr);
      if (!(nr >= 1.17549435e-38f) || !(nr <= 3.40282347e38f) || !(inv < __builtin_huge_valf())) {
        ++bad;
        continue;
      }
      mn = std::min(mn, __float_as_uint(nr));
      scale = inv;
    }
    for (int d = lane; d < dim; d += 64) m = std::max(m, f2u_abs(rows[r * dim + d] * scale));
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = std::max(m, (uint32_t)__shfl_xor((int)m, off));
  if (lane == 0) {
    red[0][wave] = m;
    red[1][wave] = bad;
    red[2][wave] = mn;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; ++w) {
      red[0][0] = std::max(red[0][0], red[0][w]);
      red[1][0] += red[1][w];
      red[2][0] = std::min(red[2][0], red[2][w]);
    }
    atomicMax(&stats[0], red[0][0]);
    if (red[1][0]) atomicAdd(&stats[1], red[1][0]);
    atomicMin(&stats[2], red[2][0]);
  }
}

// Blocked fp16 rows: block b (rows 32b..32b+31), k-step kb, lane l holds the
// 8 halves of row 32b + l%32, dims 16kb + 8(l/32) + 0..7 (zero beyond n or
// dim): the A operand of one v_mfma_f32_32x32x16_f16, 1 KiB contiguous.
__global__ __launch_bounds__(256) void rows_to_h16_kernel(const float* __restrict__ rows, uint64_t n, int dim,
                                                          int kb, const float* __restrict__ rn, int cosine,
                                                          int ex, v8h* __restrict__ out, uint64_t units) {
  const uint64_t u = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= units) return;
  const int l = (int)(u & 63);
  const uint64_t bk = u >> 6;  // b * kb + kstep
  const uint64_t b = bk / (uint64_t)kb;
  const int ks = (int)(bk - b * (uint64_t)kb);
  const uint64_t r = b * 32 + (uint64_t)(l & 31);
  const int d0 = 16 * ks + 8 * (l >> 5);
  v8h h;
  float scale = 1.0f;
  if (r < n && cosine) scale = 1.0f / __builtin_sqrtf(rn[r]);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int d = d0 + t;
    const float v = (r < n && d < dim) ? ldexpf(rows[r * dim + d] * scale, ex) : 0.0f;
    h[t] = (_Float16)v;
  }
  out[u] = h;
}

__global__ void pad_norms_kernel(const float* __restrict__ rn, uint64_t n, uint64_t npad, float* __restrict__ out) {
  const uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < npad) out[i] = i < n ? rn[i] : 0.0f;
}

// ---- queries (per pass) -------------------------------------------------------

// One wave per query slot of the padded tiles: blocked fp16 operand (the B
// operand: lane l holds query 32t + l%32, dims 16kb + 8(l/32) + 0..7), its
// exponent, tau = +inf (-inf and forced for a query the fp16 path cannot
// take).  Cosine: the reference divides by sqrt(qn * rn), which
// must stay clear of underflow and overflow for every row (rn in [rnmin,
// rnmax]) for the normalised product to stand for it.
__global__ __launch_bounds__(64) void queries_to_h16_kernel(const float* __restrict__ qs, uint64_t nq, int dim,
                                                            int kb, const float* __restrict__ qn, int cosine,
                                                            float rnmin, float rnmax, int ex,
                                                            v8h* __restrict__ q16, int* __restrict__ qexp,
                                                            float* __restrict__ tau, int* __restrict__ force) {
  const uint64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  const bool real = q < nq;
  float scale = 1.0f;
  bool bad = false;
  if (real && cosine) {
    const float n2 = qn[q];
    scale = 1.0f / __builtin_sqrtf(n2);
    bad = !(n2 >= 1.17549435e-38f) || !(scale < __builtin_huge_valf()) ||
          !(n2 * rnmin >= 7.8886091e-31f) || !(n2 * rnmax <= 1.2676506e30f);  // 2^-100, 2^100
  }
  uint32_t m = 0;
  if (real && !bad)
    for (int d = lane; d < dim; d += 64) m = std::max(m, f2u_abs(qs[q * dim + d] * scale));
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = std::max(m, (uint32_t)__shfl_xor((int)m, off));
  const float maxabs = __uint_as_float(m);
  bad = bad || !(maxabs < __builtin_huge_valf());
  const int e = scale_exp(maxabs);
  // the unscaling factor 2^-(e + ex) must stay a normal float
  bad = bad || e + ex > 120 || e + ex < -120;
  const uint64_t tile = q >> 5;
  const int ql = (int)(q & 31);
  for (int d = lane; d < 16 * kb; d += 64) {
    const float v = (real && !bad && d < dim) ? ldexpf(qs[q * dim + d] * scale, e) : 0.0f;
    const int ks = d >> 4, half = (d >> 3) & 1, t = d & 7;
    reinterpret_cast<_Float16*>(q16)[(((tile * kb + ks) * 64) + ql + 32 * half) * 8 + t] = (_Float16)v;
  }
  if (lane == 0 && real) {
    qexp[q] = e;
    tau[q] = bad ? -__builtin_huge_valf() : __builtin_huge_valf();
    force[q] = bad ? 1 : 0;
  }
}

// ---- the screening kernel ---------------------------------------------------------

struct Screen16Args {
  const v8h* x16;
  uint64_t n, nblk;
  const float* rn16;  // [nblk*32] squared norms, zero-padded (L2 only)
  const v8h* q16;     // [qtiles][kb][64]
  uint64_t nq;
  const float* qn;    // [nq] (L2 only)
  const int* qexp;    // [nq]
  int xexp;
  const float* tau;   // [nq]
  // append buffers, one per (query, chunk, half wave): sb = (q*nchunks +
  // chunk)*2 + half holds scnt[sb] entries (the first kSub of them stored)
  // at sbuf[sb*kSub ..]: (screening value bits, row)
  uint32_t* scnt;
  uint2* sbuf;
  uint32_t nchunks;
  uint64_t bstride, nsel, chunk_blocks;
};

enum { kScrDot = 0, kScrCos = 1, kScrL2 = 2 };

// Workgroup: 4 waves x T query tiles of 32 (128T queries) over a chunk of
// the selected blocks.  The queries' operands stay in registers; each stage
// of SB = 32/KB row blocks goes through LDS once and feeds every wave.  Per
// block and tile a lane holds 16 products of its query (32t + lane%32) with
// rows 8(r/4) + 4(lane/32) + r%4 and tests them against its threshold.
template <int MET, int KB, int T>
// Dot and cosine up to 256 dimensions fit three waves per SIMD (168 VGPRs).
__global__ __launch_bounds__(kT16)
__attribute__((amdgpu_waves_per_eu((MET != kScrL2 && KB <= 16) ? 3 : 1, 8))) void screen16_kernel(Screen16Args a) {
  constexpr int SB = (kStageKiB / KB) > 0 ? kStageKiB / KB : 1;
  __shared__ v8h stage[SB * KB * 64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const uint64_t tile0 = (uint64_t)blockIdx.x * (4 * T) + (uint64_t)wave * T;

  v8h bq[T][KB];
  float thr[T], fac[T], qnv[T];
  uint64_t qidx[T], sbase[T];
  uint32_t cnt[T];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint64_t tile = tile0 + t;
    const uint64_t q = tile * 32 + (uint64_t)(lane & 31);
    qidx[t] = q;
    sbase[t] = ((q * a.nchunks + blockIdx.y) * 2 + (uint64_t)h) * kSub;
    cnt[t] = 0;
    const bool real = q < a.nq;
#pragma unroll
    for (int ks = 0; ks < KB; ++ks) bq[t][ks] = a.q16[(tile * KB + ks) * 64 + lane];
    const float tq = real ? a.tau[q] : -__builtin_huge_valf();
    const int e = (real ? a.qexp[q] : 0) + a.xexp;
    if constexpr (MET == kScrDot) {
      thr[t] = ldexpf(-tq, e);   // -acc * 2^-e <= tau  <=>  acc >= -tau * 2^e
      fac[t] = -ldexpf(1.0f, -e);
    } else if constexpr (MET == kScrCos) {
      thr[t] = tq;
      fac[t] = -ldexpf(1.0f, -e);  // v = 1 - acc * 2^-e, one rounding
    } else {
      thr[t] = tq;
      fac[t] = -ldexpf(2.0f, -e);  // v = (qn + rn) - 2 * acc * 2^-e
      qnv[t] = real ? a.qn[q] : 0.0f;
    }
  }

  const uint64_t j0 = (uint64_t)blockIdx.y * a.chunk_blocks;
  const uint64_t j1 = std::min<uint64_t>(a.nsel, j0 + a.chunk_blocks);  // > j0: no empty chunks
  constexpr int kUnits = SB * KB * 64;
  constexpr int kPer = (kUnits + kT16 - 1) / kT16;
  // The next stage's loads are issued before the current stage is computed.
  // Blocks past the chunk's end re-read its last block (never computed).
  v8h pre[kPer];
  auto fetch = [&](uint64_t js) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * kT16;
      if (kUnits % kT16 == 0 || u < kUnits) {
        const int bs = u / (KB * 64);
        const uint64_t j = std::min<uint64_t>(js + (uint64_t)bs, j1 - 1);
        pre[i] = a.x16[(j * a.bstride * KB) * 64 + (uint64_t)(u - bs * KB * 64)];
      }
    }
  };
  fetch(j0);
  for (uint64_t js = j0; js < j1; js += SB) {
    __syncthreads();  // the previous stage is consumed
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int u = tid + i * kT16;
      if (kUnits % kT16 == 0 || u < kUnits) stage[u] = pre[i];
    }
    __syncthreads();
    if (js + SB < j1) fetch(js + SB);
#pragma unroll 1
    for (int bs = 0; bs < SB; ++bs) {
      const uint64_t j = js + (uint64_t)bs;
      if (j >= j1) break;
      const uint64_t gb = j * a.bstride;
      v16f acc[T];
#pragma unroll
      for (int t = 0; t < T; ++t) acc[t] = v16f{};
#pragma unroll
      for (int ks = 0; ks < KB; ++ks) {
        const v8h av = stage[(bs * KB + ks) * 64 + lane];
#pragma unroll
        for (int t = 0; t < T; ++t) acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bq[t][ks], acc[t], 0, 0, 0);
      }
      const uint64_t rbase = gb * 32 + (uint64_t)(4 * h);
      float rnv[16];
      if constexpr (MET == kScrL2) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 v4 = *reinterpret_cast<const float4*>(a.rn16 + rbase + 8 * g);
          rnv[4 * g] = v4.x;
          rnv[4 * g + 1] = v4.y;
          rnv[4 * g + 2] = v4.z;
          rnv[4 * g + 3] = v4.w;
        }
      }
#pragma unroll
      for (int t = 0; t < T; ++t) {
        // hot test: one compare (a ballot) per value; appends only for the
        // values some lane passes (the screening value is recomputed there,
        // not kept in registers)
        auto value = [&](int r) {
          if constexpr (MET == kScrDot) return acc[t][r];
          else if constexpr (MET == kScrCos) return __builtin_fmaf(acc[t][r], fac[t], 1.0f);
          else return __builtin_fmaf(acc[t][r], fac[t], qnv[t] + rnv[r]);
        };
        uint64_t mk[16];
        uint64_t any = 0;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float v = value(r);
          mk[r] = __ballot((MET == kScrDot) ? v >= thr[t] : v <= thr[t]);
          any |= mk[r];
        }
        if (any == 0) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (mk[r] == 0) continue;
          // row of value r: 8(r/4) + 4h + r%4 within the block; rows past n
          // (the last block only) never pass
          const uint32_t row = (uint32_t)(rbase + 8 * (r >> 2) + (r & 3));
          if (((mk[r] >> lane) & 1u) && row < a.n) {
            if (cnt[t] < kSub) {
              const float v = (MET == kScrDot) ? value(r) * fac[t] : value(r);
              a.sbuf[sbase[t] + cnt[t]] = make_uint2(__float_as_uint(v), row);
            }
            ++cnt[t];
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < T; ++t)
    if (qidx[t] < a.nq) a.scnt[sbase[t] / kSub] = cnt[t];
}

// ---- per-stage selection --------------------------------------------------------

// One wave per query over its nsub append buffers.  Middle stage: tau = the
// m-th smallest value stored (kept when fewer arrived; a buffer that
// overflowed dropped entries, and the m-th of the rest still has m rows at
// or below it).  Last stage: the kp smallest (value, row) pairs as
// candidates, abound = the kp-th value (every row outside screens at or above
// it) or tau when fewer arrived; an overflowing or forced query gets cand
// count kForceExact.
template <int R>
__global__ __launch_bounds__(64) void select16_kernel(const uint32_t* __restrict__ scnt,
                                                      const uint2* __restrict__ sbuf, uint32_t nsub,
                                                      float* __restrict__ tau, int m, int final_stage, int kp,
                                                      const int* __restrict__ force, float* __restrict__ cand_d,
                                                      uint64_t* __restrict__ cand_k, uint32_t* __restrict__ cand_c,
                                                      float* __restrict__ abound) {
  const uint64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  WaveTopK<R> tk;
  tk.init(final_stage ? kp : m);
  uint32_t stored = 0;
  bool over = false;
  for (uint32_t s0 = 0; s0 < nsub; s0 += 64) {
    const uint32_t s = s0 + (uint32_t)lane;
    const uint32_t c = s < nsub ? scnt[q * nsub + s] : 0u;
    over = over || __ballot(c > kSub) != 0;
    const uint32_t ce = std::min(c, kSub);
    uint32_t cmax = ce;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) cmax = std::max(cmax, (uint32_t)__shfl_xor((int)cmax, off));
    const uint2* __restrict__ b = sbuf + (q * nsub + s) * kSub;
    for (uint32_t i = 0; i < cmax; ++i) {
      const bool in = i < ce;
      const uint2 e = in ? b[i] : make_uint2(0u, 0u);
      tk.offer(in ? __uint_as_float(e.x) : f_inf(), in ? e.y : kNoPos);
    }
    uint32_t sum = ce;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) sum += (uint32_t)__shfl_xor((int)sum, off);
    stored += sum;
  }
  const float t_old = tau[q];
  if (!final_stage) {
    if (stored >= (uint32_t)m && lane == 0) tau[q] = tk.tau;
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = r * 64 + lane;
    if (s < kp) {
      cand_d[q * kp + s] = tk.d[r];
      cand_k[q * kp + s] = tk.p[r] == kNoPos ? ~0ull : (uint64_t)tk.p[r];
    }
  }
  if (lane == 0) {
    const bool forced = force[q] != 0 || over;
    cand_c[q] = forced ? kForceExact : std::min<uint32_t>(stored, (uint32_t)kp);
    abound[q] = stored >= (uint32_t)kp ? tk.tau : t_old;
  }
}

template <int MET, int KB>
void* pick16_t() {
  if constexpr (KB <= 8) return (void*)screen16_kernel<MET, KB, 2>;
  else return (void*)screen16_kernel<MET, KB, 1>;
}

template <int MET>
void* pick16(int kb) {
  switch (kb) {
    case 4: return pick16_t<MET, 4>();
    case 6: return pick16_t<MET, 6>();
    case 8: return pick16_t<MET, 8>();
    case 12: return pick16_t<MET, 12>();
    case 16: return pick16_t<MET, 16>();
    case 24: return pick16_t<MET, 24>();
    case 32: return pick16_t<MET, 32>();
  }
  return nullptr;
}

int tiles_per_wave(int kb) { return kb <= 8 ? 2 : 1; }

unsigned cdiv(uint64_t a, uint64_t b) { return (unsigned)((a + b - 1) / b); }

__global__ void zero_counter(uint32_t* p) { *p = 0; }

}  // namespace

// k-steps of 16 dimensions: the next supported count at or above dim/16.
int h16_ksteps(int dim) {
  const int need = (dim + 15) / 16;
  for (int kb : {4, 6, 8, 12, 16, 24, 32})
    if (need <= kb) return kb;
  return 0;
}

void H16Rows::build(const float* rows, const float* row_norm, uint64_t n, int dim, int metric,
                    hipStream_t s) {
  ok = false;
  n_ = n;
  dim_ = dim;
  kb = h16_ksteps(dim);
  if (n == 0 || kb == 0 || dim % 4 != 0) return;
  if (metric == FDB_METRIC_MANHATTAN) return;
  const int cosine = metric == FDB_METRIC_COSINE ? 1 : 0;
  stats_.reserve(3);
  hipLaunchKernelGGL(init_stats, dim3(1), dim3(1), 0, s, stats_.p);
  FDB_HIP(hipGetLastError());
  hipLaunchKernelGGL(rows_absmax_kernel, dim3(std::min<unsigned>(2048, cdiv(n, 4))), dim3(256), 0, s, rows, n,
                     dim, row_norm, cosine, stats_.p);
  FDB_HIP(hipGetLastError());
  uint32_t st[3];
  FDB_HIP(hipMemcpyAsync(st, stats_.p, sizeof(st), hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  float maxabs;
  std::memcpy(&maxabs, &st[0], 4);
  std::memcpy(&rnmin, &st[2], 4);
  // zero, denormal or non-finite norms (cosine), non-finite values
  if (st[1] != 0 || !std::isfinite(maxabs)) return;
  int e = 0;
  if (maxabs > 0.0f) {
    int ee;
    (void)std::frexp(maxabs, &ee);
    e = 14 - ee;
  }
  if (e > 100 || e < -100) return;
  xexp = e;
  nblk = (n + 31) / 32;
  const uint64_t units = nblk * (uint64_t)kb * 64;
  x16_.reserve(units * 8);
  hipLaunchKernelGGL(rows_to_h16_kernel, dim3(cdiv(units, 256)), dim3(256), 0, s, rows, n, dim, kb, row_norm,
                     cosine, e, reinterpret_cast<v8h*>(x16_.p), units);
  FDB_HIP(hipGetLastError());
  if (metric == FDB_METRIC_EUCLIDEAN || metric == FDB_METRIC_EUCLIDEAN_SQUARED) {
    rn16_.reserve(nblk * 32);
    hipLaunchKernelGGL(pad_norms_kernel, dim3(cdiv(nblk * 32, 256)), dim3(256), 0, s, row_norm, n, nblk * 32,
                       rn16_.p);
    FDB_HIP(hipGetLastError());
  }
  ok = true;
}

bool FlatSearcher::screenable16(const H16Rows& h, int metric, uint32_t k) {
  return h.ok && screenable(metric, h.dim_, k) && metric != FDB_METRIC_MANHATTAN;
}

void FlatSearcher::screen16(const FlatRows& x, const H16Rows& h, int metric, const float* d_qs,
                            const float* q_norm, uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists,
                            uint32_t* d_counts, hipStream_t s) {
  if (!screenable16(h, metric, k)) throw Error(FDB_ERR_UNSUPPORTED, "fp16 screening does not apply");
  const int kp = (k + 16 <= 64) ? 64 : 128;
  const int kb = h.kb;
  const int T = tiles_per_wave(kb);
  const int met = metric == FDB_METRIC_DOT_PRODUCT ? kScrDot : (metric == FDB_METRIC_COSINE ? kScrCos : kScrL2);
  void* fn = met == kScrDot ? pick16<kScrDot>(kb) : (met == kScrCos ? pick16<kScrCos>(kb) : pick16<kScrL2>(kb));
  if (!fn) throw Error(FDB_ERR_UNSUPPORTED, "no fp16 screening kernel for this dimension");

  // The ladder of block counts, last = all blocks: an 8x step into the last
  // stage (its threshold is the 32nd value of a 1/8 sample: about 256 rows
  // of every block pass it, with a spread of about 1/sqrt(32)), 32x steps
  // before, down to a first stage of at most 32 blocks.
  std::vector<uint64_t> ladder{h.nblk};
  if (h.nblk > 32) ladder.insert(ladder.begin(), (h.nblk + 7) / 8);
  while (ladder.front() > 32) ladder.insert(ladder.begin(), (ladder.front() + 31) / 32);

  // balanced passes of at most kSlice queries
  const uint64_t passes = (nq + kSlice - 1) / kSlice;
  const uint64_t slice = (nq + passes - 1) / passes;
  const uint64_t qtiles_max = (slice + 31) / 32;
  const uint64_t groups_max = (qtiles_max + 4 * T - 1) / (4 * T);
  // Chunks per stage: about 2048 workgroups, within the append budget; a
  // small stage (the first, or any of at most 64 blocks, where tau may still
  // be +inf) takes at most 4 blocks per chunk so that every row of a half
  // wave's 64 fits its buffer.
  // Workgroups resident on the whole GPU at once: the grid is sized in whole
  // rounds of them (a partial last round measured ~12% slower).
  int occ = 0, cus = 0, dev = 0;
  FDB_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, (const void*)fn, kT16, 0));
  FDB_HIP(hipGetDevice(&dev));
  FDB_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const uint64_t resident = std::max<uint64_t>(1, (uint64_t)std::max(occ, 1) * (uint64_t)std::max(cus, 1));
  auto chunks = [&](uint64_t nsel, uint64_t groups, uint64_t m, bool small) {
    const uint64_t room = std::max<uint64_t>(1, kSubBudget / (m * 2 * kSub));
    const uint64_t rounds = room * groups / resident;  // whole rounds the buffers allow
    uint64_t want = rounds >= 1 ? std::max<uint64_t>(1, rounds * resident / groups) : room;
    want = std::min(want, room);
    uint64_t cb = (nsel + want - 1) / want;
    if (small) cb = std::min<uint64_t>(cb, 4);
    cb = std::max<uint64_t>(cb, 1);
    return std::make_pair(cb, (nsel + cb - 1) / cb);
  };
  // buffer sizes: the largest over every pass and stage (a shorter pass has
  // fewer query groups and may take more chunks)
  uint64_t max_subs = 1;
  for (uint64_t q0 = 0; q0 < nq; q0 += slice) {
    const uint64_t m = std::min(slice, nq - q0);
    const uint64_t groups = ((m + 31) / 32 + 4 * T - 1) / (4 * T);
    for (size_t st = 0; st < ladder.size(); ++st)
      max_subs = std::max(max_subs, m * 2 * chunks(ladder[st], groups, m, st == 0 || ladder[st] <= 64).second);
  }
  q16_.reserve((groups_max * 4 * (uint64_t)T) * (uint64_t)kb * 64 * 8);
  qexp_.reserve(slice);
  tau_.reserve(slice);
  force_.reserve(slice);
  count_.reserve(max_subs);
  buf_.reserve(max_subs * kSub);
  cand_d_.reserve(slice * kp);
  cand_k_.reserve(slice * kp);
  cand_c_.reserve(slice);
  abound_.reserve(slice);
  flags_.reserve(nq);
  fallbacks_.reserve(1);
  hipLaunchKernelGGL(zero_counter, dim3(1), dim3(1), 0, s, fallbacks_.p);
  FDB_HIP(hipGetLastError());

  for (uint64_t q0 = 0; q0 < nq; q0 += slice) {
    const uint64_t m = std::min(slice, nq - q0);
    const uint64_t qtiles = (m + 31) / 32;
    // tiles past the last one that a workgroup reads are zero queries
    const uint64_t groups = (qtiles + 4 * T - 1) / (4 * T);
    const uint64_t slots = groups * 4 * T * 32;
    hipLaunchKernelGGL(queries_to_h16_kernel, dim3((unsigned)slots), dim3(64), 0, s, d_qs + q0 * h.dim_, m,
                       h.dim_, kb, q_norm + q0, met == kScrCos ? 1 : 0, h.rnmin, x.rnmax, h.xexp,
                       reinterpret_cast<v8h*>(q16_.p), qexp_.p, tau_.p, force_.p);
    FDB_HIP(hipGetLastError());
    for (size_t st = 0; st < ladder.size(); ++st) {
      const bool last = st + 1 == ladder.size();
      const uint64_t nsel = ladder[st];
      const auto [cb, nch] = chunks(nsel, groups, m, st == 0 || nsel <= 64);
      Screen16Args a{};
      a.x16 = reinterpret_cast<const v8h*>(h.x16());
      a.n = h.n_;
      a.nblk = h.nblk;
      a.rn16 = h.rn16();
      a.q16 = reinterpret_cast<const v8h*>(q16_.p);
      a.nq = m;
      a.qn = q_norm + q0;
      a.qexp = qexp_.p;
      a.xexp = h.xexp;
      a.tau = tau_.p;
      a.scnt = count_.p;
      a.sbuf = buf_.p;
      a.nchunks = (uint32_t)nch;
      a.bstride = last ? 1 : h.nblk / nsel;
      a.nsel = nsel;
      a.chunk_blocks = cb;
      void* args[] = {(void*)&a};
      FDB_HIP(hipLaunchKernel(fn, dim3((unsigned)groups, (unsigned)nch), dim3(kT16), args, 0, s));
      const uint32_t nsub = (uint32_t)(2 * nch);
      if (!last) {
        // rank for the next threshold: about 256 rows of the next stage pass
        // it; 32 at least before the last stage, whose threshold bounds the
        // rows it leaves out
        const uint64_t ratio = std::max<uint64_t>(1, ladder[st + 1] / nsel);
        const uint64_t lo = st + 2 == ladder.size() ? 32 : 8;
        const int rank = (int)std::clamp<uint64_t>(256 / ratio, lo, 64);
        hipLaunchKernelGGL(select16_kernel<1>, dim3((unsigned)m), dim3(64), 0, s, count_.p, buf_.p, nsub, tau_.p,
                           rank, 0, kp, force_.p, cand_d_.p, cand_k_.p, cand_c_.p, abound_.p);
      } else if (kp == 64) {
        hipLaunchKernelGGL(select16_kernel<1>, dim3((unsigned)m), dim3(64), 0, s, count_.p, buf_.p, nsub, tau_.p, 0,
                           1, kp, force_.p, cand_d_.p, cand_k_.p, cand_c_.p, abound_.p);
      } else {
        hipLaunchKernelGGL(select16_kernel<2>, dim3((unsigned)m), dim3(64), 0, s, count_.p, buf_.p, nsub, tau_.p, 0,
                           1, kp, force_.p, cand_d_.p, cand_k_.p, cand_c_.p, abound_.p);
      }
      FDB_HIP(hipGetLastError());
    }
    RescoreArgs r{};
    r.queries = d_qs + q0 * x.dim;
    r.dim = x.dim;
    r.rows = x.rows;
    r.row_norm = x.row_norm;
    r.q_norm = q_norm + q0;
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
    r.abound = abound_.p;
    r.bkind = kBoundH16;
    r.n = x.n;
    FDB_HIP(launch_rescore(r, m, s));
  }
  exact(x, metric, d_qs, q_norm, nq, k, d_ids, d_dists, d_counts, s, flags_.p);
}

}  // namespace fdb
