// forge-db query-path kernels for gfx950 (wave64).
//
// coarse_select_kernel  exact squared-L2 query-to-centroid distances in the
//                       reference's AVX2 order + nprobe selection in registers
//                       (src/index/ivf_pq.rs:538-553, src/index/ivf.rs:164-177)
// ivfpq_scan_kernel     per query: residual LUTs in LDS (src/pq.rs:149-189),
//                       ADC over the probed lists' codes (src/pq.rs:218-485),
//                       wave64 top-k and merge (src/index/ivf_pq.rs:590-677,
//                       :850-1047)
// kmeans_update_kernel, pq_encode_kernel, transpose kernels: build side
//                       (src/kmeans.rs:87-193, src/pq.rs:114-139)
#include "fdb_kernels.hpp"

#include <algorithm>

#include "fdb_device.hpp"

namespace fdb {

namespace {

constexpr int kThreads = 256;
constexpr int kCoarseTQ = 4;                 // queries per wave
constexpr int kCoarseQB = 4 * kCoarseTQ;     // queries per workgroup (4 waves)
// below this many query tiles (two per CU) the centroids are split into
// parts: at 100 queries four parts ran 2-3.5x faster, at 10,000 queries (625
// tiles) one part was 5-30% faster, every part paying its own list fill
constexpr uint64_t kCoarseTargetWG = 512;
// bound on the partial-list workspace, in (distance, centroid) entries
constexpr uint64_t kCoarsePartEntries = 1ull << 24;

// ---------------------------------------------------------------------------
// Coarse selection.  A workgroup takes kCoarseQB queries, each wave 4 of
// them, and sweeps one part of the centroids (blockIdx.y: centroids
// [y*part_len, (y+1)*part_len), part_len a multiple of 256; all of them when
// gridDim.y = 1) 256 at a time, so the four waves read the same centroid
// values and a small batch can still fill the GPU: lane L holds centroids
// c..c+3 (c = base + 4L).  For lane l of the reference's 8 FMA lanes it
// walks rows l*d8 .. l*d8+d8-1 of centT: one coalesced float4 of centroid
// values and one wave-uniform (broadcast) float4 of the wave's 4 query values
// per row feed 16 independent FMA chains; each finished lane chain is added
// to the running total left to right, then the tail rows are added as
// separate multiply and add.  The 16 distances go straight from registers
// into the wave's 4 WaveTopK lists through per-query LDS queues
// (offer_queued), so a list is merged once per 64 passing candidates rather
// than at every offer.  centT rows have ldc >= nlist (a
// multiple of 256) entries; columns >= nlist are never selected.  With one
// part the lists are the result; with several, each part's list goes to
// part_d / part_k [nq][parts][nsel] and coarse_merge_kernel selects from them.
// ---------------------------------------------------------------------------
// D8T: compile-time floor(dim / 8) (0 = runtime), so one lane's rows can be
// loaded before any is used.
template <int R, int D8T>
__global__ __launch_bounds__(kThreads) void coarse_select_kernel(
    const float* __restrict__ queries, uint64_t nq, int dim, const float* __restrict__ centT,
    int ldc, int nlist, int nsel, int32_t* __restrict__ out_lists, float* __restrict__ out_dists,
    int* __restrict__ err_flag, int part_len, float* __restrict__ part_d,
    uint32_t* __restrict__ part_k, const int* __restrict__ only) {
  extern __shared__ float qsT[];  // [dim][QB], rows permuted
  __shared__ uint2 s_queue[kThreads / 64][kCoarseTQ][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint64_t q0 = (uint64_t)blockIdx.x * kCoarseQB;
  const int d8 = D8T ? D8T : dim / 8;
  if (only) {
    // only the workgroups holding a flagged query run; the others' lists
    // are already written (and would be the same).  Lane i < kCoarseQB of
    // each wave reads query i's flag: one load and a ballot, not a chain of
    // loads.
    static_assert(kCoarseQB <= 64, "a wave reads the workgroup's flags");
    const bool f = lane < kCoarseQB && q0 + lane < nq && only[q0 + lane] != 0;
    if (__ballot(f) == 0) return;
  }

  for (int e = tid; e < kCoarseQB * dim; e += kThreads) {
    const int qq = e / dim;
    const int d = e - qq * dim;
    const int row = (d >= 8 * d8) ? d : (d % 8) * d8 + d / 8;
    qsT[row * kCoarseQB + qq] = (q0 + qq < nq) ? queries[(q0 + qq) * (uint64_t)dim + d] : 0.0f;
  }
  WaveTopK<R> tk[kCoarseTQ];
  int qn[kCoarseTQ];
#pragma unroll
  for (int t = 0; t < kCoarseTQ; ++t) {
    tk[t].init(nsel);
    qn[t] = 0;
  }
  bool saw_nan = false;
  __syncthreads();

  const float* __restrict__ qw = qsT + wave * kCoarseTQ;
  const int c_beg = (int)blockIdx.y * part_len;
  const int c_end = min(nlist, c_beg + part_len);
  for (int base = c_beg; base < c_end; base += 256) {
    const int c = base + 4 * lane;
    float tot[kCoarseTQ][4];
#pragma unroll
    for (int t = 0; t < kCoarseTQ; ++t)
#pragma unroll
      for (int u = 0; u < 4; ++u) tot[t][u] = 0.0f;
#pragma unroll 1
    for (int l = 0; l < 8 && d8 > 0; ++l) {
      float ch[kCoarseTQ][4];
#pragma unroll
      for (int t = 0; t < kCoarseTQ; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) ch[t][u] = 0.0f;
      if constexpr (D8T > 0) {
        float4 cvs[D8T];
#pragma unroll
        for (int i = 0; i < D8T; ++i)
          cvs[i] = *reinterpret_cast<const float4*>(centT + (uint64_t)(l * D8T + i) * ldc + c);
#pragma unroll
        for (int i = 0; i < D8T; ++i) {
          const float4 qv = *reinterpret_cast<const float4*>(qw + (l * D8T + i) * kCoarseQB);
          const float cva[4] = {cvs[i].x, cvs[i].y, cvs[i].z, cvs[i].w};
          const float qva[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
          for (int t = 0; t < kCoarseTQ; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float df = qva[t] - cva[u];
              ch[t][u] = __builtin_fmaf(df, df, ch[t][u]);
            }
        }
      } else {
#pragma unroll 2
        for (int i = 0; i < d8; ++i) {
          const int row = l * d8 + i;
          const float4 cv = *reinterpret_cast<const float4*>(centT + (uint64_t)row * ldc + c);
          const float4 qv = *reinterpret_cast<const float4*>(qw + row * kCoarseQB);
          const float cva[4] = {cv.x, cv.y, cv.z, cv.w};
          const float qva[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
          for (int t = 0; t < kCoarseTQ; ++t)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
              const float df = qva[t] - cva[u];
              ch[t][u] = __builtin_fmaf(df, df, ch[t][u]);
            }
        }
      }
#pragma unroll
      for (int t = 0; t < kCoarseTQ; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) tot[t][u] = (l == 0) ? ch[t][u] : tot[t][u] + ch[t][u];
    }
    for (int row = 8 * d8; row < dim; ++row) {
      const float4 cv = *reinterpret_cast<const float4*>(centT + (uint64_t)row * ldc + c);
      const float4 qv = *reinterpret_cast<const float4*>(qw + row * kCoarseQB);
      const float cva[4] = {cv.x, cv.y, cv.z, cv.w};
      const float qva[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
      for (int t = 0; t < kCoarseTQ; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const float df = qva[t] - cva[u];
          tot[t][u] = tot[t][u] + df * df;
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool in = c + u < c_end;
#pragma unroll
      for (int t = 0; t < kCoarseTQ; ++t) {
        const float dv = tot[t][u];
        if (in && dv != dv) saw_nan = true;
        tk[t].offer_queued(dv, (uint32_t)(c + u), in, s_queue[wave][t], qn[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < kCoarseTQ; ++t) tk[t].flush(s_queue[wave][t], qn[t]);

  const bool parts = gridDim.y > 1;
#pragma unroll
  for (int t = 0; t < kCoarseTQ; ++t) {
    const uint64_t q = q0 + wave * kCoarseTQ + t;
    if (q >= nq) continue;
    const uint64_t o = parts ? (q * gridDim.y + blockIdx.y) * nsel : q * nsel;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int s = r * 64 + lane;
      if (s < nsel) {
        if (parts) {
          part_d[o + s] = tk[t].d[r];
          part_k[o + s] = tk[t].p[r];
        } else {
          out_lists[o + s] = (int32_t)tk[t].p[r];
          if (out_dists) out_dists[o + s] = tk[t].d[r];
        }
      }
    }
  }
  if (saw_nan && err_flag) atomicOr(err_flag, 1);
}

// One wave per query: the nsel smallest (distance, centroid) pairs of its
// `parts` partial lists (entries without a centroid are (+inf, kNoPos)).
template <int R>
__global__ __launch_bounds__(kThreads) void coarse_merge_kernel(
    const float* __restrict__ part_d, const uint32_t* __restrict__ part_k, uint64_t nq, int parts,
    int nsel, int32_t* __restrict__ out_lists, float* __restrict__ out_dists) {
  const int lane = threadIdx.x & 63;
  const uint64_t q = (uint64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (q >= nq) return;
  WaveTopK<R> tk;
  tk.init(nsel);
  const int total = parts * nsel;
  const float* pd = part_d + q * total;
  const uint32_t* pk = part_k + q * total;
  for (int b = 0; b < total; b += 64) {
    const int e = b + lane;
    tk.offer(e < total ? pd[e] : f_inf(), e < total ? pk[e] : kNoPos);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = r * 64 + lane;
    if (s < nsel) {
      out_lists[q * nsel + s] = (int32_t)tk.p[r];
      if (out_dists) out_dists[q * nsel + s] = tk.d[r];
    }
  }
}

template <int R>
hipError_t launch_coarse_t(const float* queries, uint64_t nq, int dim, const float* centT, int ldc,
                           int nlist, int nsel, int32_t* out_lists, float* out_dists, int* err_flag,
                           int parts, float* part_d, uint32_t* part_k, const int* only, hipStream_t stream) {
  const size_t lds = sizeof(float) * (size_t)kCoarseQB * dim;
  void (*fn)(const float*, uint64_t, int, const float*, int, int, int, int32_t*, float*, int*, int,
             float*, uint32_t*, const int*) =
      dim / 8 == 16 ? coarse_select_kernel<R, 16>
                    : (dim / 8 == 12 ? coarse_select_kernel<R, 12> : coarse_select_kernel<R, 0>);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
  }
  const uint64_t blocks = (nq + kCoarseQB - 1) / kCoarseQB;
  const int part_len = (ldc / 256 + parts - 1) / parts * 256;
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks, (unsigned)parts), dim3(kThreads), lds, stream,
                     queries, nq, dim, centT, ldc, nlist, nsel, out_lists, out_dists, err_flag,
                     part_len, part_d, part_k, only);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || parts == 1) return e;
  hipLaunchKernelGGL(coarse_merge_kernel<R>, dim3((unsigned)((nq + 3) / 4)), dim3(kThreads), 0,
                     stream, part_d, part_k, nq, parts, nsel, out_lists, out_dists);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Fused IVF-PQ scan.  One workgroup per query.  The probed lists are taken G
// at a time: the G residuals q - c_p go to LDS, then thread t (one per
// codeword) builds entry t of every subspace table for all G lists, holding
// the codeword in registers and reading the residual as a wave-uniform LDS
// broadcast, so each codebook row is fetched once per G lists.  The scan
// streams each list's codes (one code vector per lane, coalesced), sums the
// LDS table entries in the requested reference order and feeds a per-wave
// top-k; the four wave lists are merged at the end.
// ---------------------------------------------------------------------------
template <int MT>
__device__ __forceinline__ void load_code(const uint8_t* __restrict__ codes, uint32_t i,
                                          uint32_t (&w)[(MT + 3) / 4]) {
  if constexpr (MT % 16 == 0) {
    const uint4* p = reinterpret_cast<const uint4*>(codes + (uint64_t)i * MT);
#pragma unroll
    for (int t = 0; t < MT / 16; ++t) {
      const uint4 v = p[t];
      w[4 * t] = v.x;
      w[4 * t + 1] = v.y;
      w[4 * t + 2] = v.z;
      w[4 * t + 3] = v.w;
    }
  } else if constexpr (MT % 8 == 0) {
    const uint2* p = reinterpret_cast<const uint2*>(codes + (uint64_t)i * MT);
#pragma unroll
    for (int t = 0; t < MT / 8; ++t) {
      const uint2 v = p[t];
      w[2 * t] = v.x;
      w[2 * t + 1] = v.y;
    }
  } else {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(codes + (uint64_t)i * MT);
#pragma unroll
    for (int t = 0; t < MT / 4; ++t) w[t] = p[t];
  }
}

// Lists of one LUT group: code range [start, start+len) of each slot.
template <int GMAX>
struct GroupLists {
  uint32_t start[GMAX];
  uint32_t len[GMAX];
  int ng;
};

// Scan of one probed list with a compile-time LUT slot J.  Each wave takes
// batches of 64 consecutive codes (batch b = lanes b*64 .. b*64+63), waves
// striding by NW; U batches per wave are loaded before any is summed so U
// code loads are in flight.  The loads are branch-free: a batch or lane past
// the end re-reads the list's last code (len > 0) and carries key kNoPos.
// FAST: the LUT holds |cb|^2 - 2<r, cb> and base = |r|^2 is added to every
// sum; otherwise base is unused (exact mode adds nothing).
// live (nullable): bitmap over list positions; a clear bit skips the code
// (tombstones, filters).
__device__ __forceinline__ bool live_at(const uint32_t* __restrict__ live, uint32_t i) {
  return (live[i >> 5] >> (i & 31)) & 1u;
}

template <int MT, int ORDER, int R, int NW, int U, int J, int FAST>
__device__ __forceinline__ void scan_list(const float* __restrict__ lut, uint32_t start, uint32_t len,
                                          float base, uint32_t w0, int lane,
                                          const uint8_t* __restrict__ codes,
                                          const uint32_t* __restrict__ live, WaveTopK<R>& tk,
                                          uint2* queue, int& qn) {
  const uint32_t nb = (len + 63) / 64;
  const uint32_t last = start + len - 1;
  uint32_t b0 = w0;
  // Steps whose U batches hold 64 codes each need no bounds or validity
  // tests when no bitmap is given.
  if (live == nullptr) {
    const uint32_t nfull = len / 64;
    for (; b0 + (uint32_t)((U - 1) * NW) < nfull; b0 += (uint32_t)(NW * U)) {
      uint32_t w[U][(MT + 3) / 4];
#pragma unroll
      for (int u = 0; u < U; ++u)
        load_code<MT>(codes, start + (b0 + (uint32_t)(u * NW)) * 64 + (uint32_t)lane, w[u]);
      float dist[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        dist[u] = adc_sum<MT, ORDER>(lut + J * (MT * 256), w[u]);
        if constexpr (FAST) dist[u] = base + dist[u];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        tk.offer_queued(dist[u], start + (b0 + (uint32_t)(u * NW)) * 64 + (uint32_t)lane, true, queue,
                        qn);
    }
  }
  for (; b0 < nb; b0 += (uint32_t)(NW * U)) {
    uint32_t w[U][(MT + 3) / 4];
    uint32_t key[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t i = start + (b0 + (uint32_t)(u * NW)) * 64 + (uint32_t)lane;
      const bool in = i <= last;  // also false for a batch past nb
      const uint32_t ic = in ? i : last;
      const bool valid = in && (live == nullptr || live_at(live, ic));
      key[u] = valid ? i : kNoPos;
      load_code<MT>(codes, ic, w[u]);
    }
    float dist[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      dist[u] = adc_sum<MT, ORDER>(lut + J * (MT * 256), w[u]);
      if constexpr (FAST) dist[u] = base + dist[u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) tk.offer_queued(dist[u], key[u], key[u] != kNoPos, queue, qn);
  }
}

template <int MT, int ORDER, int R, int NW, int U, int GMAX, int J, int FAST>
__device__ __forceinline__ void scan_group(const float* __restrict__ lut, const float* __restrict__ rr,
                                           const GroupLists<GMAX>& gl, uint32_t w0, int lane,
                                           const uint8_t* __restrict__ codes,
                                           const uint32_t* __restrict__ live, WaveTopK<R>& tk,
                                           uint2* queue, int& qn) {
  if (J < gl.ng && gl.len[J] > 0)
    scan_list<MT, ORDER, R, NW, U, J, FAST>(lut, gl.start[J], gl.len[J], FAST ? rr[J] : 0.0f, w0,
                                            lane, codes, live, tk, queue, qn);
  if constexpr (J + 1 < GMAX)
    scan_group<MT, ORDER, R, NW, U, GMAX, J + 1, FAST>(lut, rr, gl, w0, lane, codes, live, tk,
                                                       queue, qn);
}

// One workgroup per query.  MT/DT: compile-time M and dsub (0 = runtime, then
// the LUTs live in dynamic LDS and each lane locates its list slot);
// NT threads; U code batches in flight per wave; at most GMAX lists per LUT
// group (G <= GMAX at run time).
template <int MT, int DT, int R, int ORDER, int NT, int U, int GMAX, int FAST>
// At most 64 VGPRs for R <= 2: 8 waves per SIMD, so four 512-thread
// workgroups (2 x 16 KiB LUTs each) fill a CU.
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(R <= 2 ? 8 : 1, 8)))
void ivfpq_scan_kernel(IvfPqScanArgs a, int G) {
  static_assert(!FAST || MT > 0, "fast LUT mode needs a specialised shape");
  constexpr int NW = NT / 64;
  // static LDS holds the LUTs + residuals, and later the wave-list merge
  // (NW lists of 64*R (distance, key) pairs)
  constexpr int SLUT = GMAX * MT * 256 + GMAX * MT * DT;
  constexpr int SLDS = (MT > 0) ? (SLUT > NW * 64 * R * 2 ? SLUT : NW * 64 * R * 2) : 1;
  __shared__ float s_static[SLDS];
  __shared__ float s_rr[GMAX];  // fast mode: |q - c_p|^2 of each list of the group
  // per-wave candidate queues (specialised shapes)
  __shared__ uint2 s_queue[MT > 0 ? NW * 64 : 1];
  extern __shared__ float s_dyn[];
  float* smem = (MT > 0) ? s_static : s_dyn;
  const int M = MT ? MT : a.M;
  const int dsub = DT ? DT : a.dsub;
  const int D = M * dsub;
  float* lut = smem;                          // [G][M][256]
  float* resid = smem + (size_t)G * M * 256;  // [G][D]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const uint32_t w0 = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const uint64_t q = blockIdx.x;
  if (a.flags && a.flags[q] == 0) return;  // the whole workgroup
  const float* __restrict__ qv = a.queries + q * D;
  const int32_t* __restrict__ pr = a.probes + q * (uint64_t)(a.pstride ? a.pstride : a.np);

  WaveTopK<R> tk;
  tk.init(a.k);
  uint2* queue = s_queue + (MT > 0 ? wave * 64 : 0);
  int qn = 0;

  for (int g0 = 0; g0 < a.np; g0 += G) {
    const int ng = min(G, a.np - g0);
    GroupLists<GMAX> gl;
    gl.ng = ng;
#pragma unroll
    for (int j = 0; j < GMAX; ++j) {
      gl.start[j] = 0;
      gl.len[j] = 0;
      if (j < ng) {
        const int p = pr[g0 + j];
        // a probe slot left empty (NaN distances) has p = -1: nothing to scan
        if (p >= 0 && p < a.nlist) {
          gl.start[j] = a.list_off[p];
          gl.len[j] = a.list_off[p + 1] - gl.start[j];
        }
      }
    }

    for (int e = tid; e < ng * D; e += NT) {
      const int j = e / D;
      const int d = e - j * D;
      const int p = pr[g0 + j];
      const float r = (p >= 0 && p < a.nlist) ? qv[d] - a.centroids[(uint64_t)p * D + d] : 0.0f;
      resid[j * D + d] = FAST ? -2.0f * r : r;  // fast mode keeps -2r (exact scaling)
    }
    __syncthreads();
    if constexpr (FAST) {
      // |r|^2 of list j by wave j: (-2r)^2 / 4, any summation order
      if (wave < ng) {
        float acc = 0.0f;
        for (int d = lane; d < D; d += 64) {
          const float v = resid[wave * D + d];
          acc = __builtin_fmaf(v, v, acc);
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
        if (lane == 0) s_rr[wave] = 0.25f * acc;
      }
    }
    // LUT: thread -> codeword tid & 255 of subspaces tid>>8, +NT/256, ...
    const int cw = tid & 255;
    for (int m = tid >> 8; m < M; m += NT / 256) {
      const float* __restrict__ cbp = a.codebooks + ((uint64_t)m * 256 + cw) * dsub;
      if constexpr (DT > 0) {
        float cbv[DT];
#pragma unroll
        for (int t = 0; t < DT; ++t) cbv[t] = cbp[t];
        if constexpr (FAST) {
          const float nrm = a.cbnorm[m * 256 + cw];
#pragma unroll
          for (int j = 0; j < GMAX; ++j)
            if (j < ng) {
              const float* __restrict__ r2 = resid + j * D + m * DT;  // -2r
              float t = nrm;
#pragma unroll
              for (int i = 0; i < DT; ++i) t = __builtin_fmaf(r2[i], cbv[i], t);
              lut[(j * M + m) * 256 + cw] = t;
            }
        } else {
#pragma unroll
          for (int j = 0; j < GMAX; ++j)
            if (j < ng) lut[(j * M + m) * 256 + cw] = l2sq_ref<DT>(resid + j * D + m * DT, cbv);
        }
      } else {
        for (int j = 0; j < ng; ++j)
          lut[(j * M + m) * 256 + cw] = l2sq_ref_rt(resid + j * D + m * dsub, cbp, dsub);
      }
    }
    __syncthreads();

    if constexpr (MT > 0) {
      scan_group<MT, ORDER, R, NW, U, GMAX, 0, FAST>(lut, s_rr, gl, w0, lane, a.codes, a.live, tk,
                                                     queue, qn);
    } else {
      // generic shape: lists one after another, one code per lane
      for (int j = 0; j < ng; ++j) {
        const int p = pr[g0 + j];
        if (p < 0 || p >= a.nlist) continue;  // uniform
        const uint32_t s = a.list_off[p], e = a.list_off[p + 1];
        const float* __restrict__ L = lut + (size_t)j * M * 256;
        for (uint32_t base = s; base < e; base += NT) {
          const uint32_t i = base + tid;
          float dist = f_inf();
          uint32_t key = kNoPos;
          if (i < e && (a.live == nullptr || live_at(a.live, i))) {
            key = i;
            dist = adc_sum_rt<ORDER>(L, a.codes + (uint64_t)i * M, M);
          }
          tk.offer(dist, key);
        }
      }
    }
    __syncthreads();
  }

  tk.flush(queue, qn);
  // merge the wave lists in wave 0
  float* md = smem;
  uint32_t* mp = reinterpret_cast<uint32_t*>(smem + NW * 64 * R);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    md[wave * 64 * R + r * 64 + lane] = tk.d[r];
    mp[wave * 64 * R + r * 64 + lane] = tk.p[r];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < NW; ++w)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int s = w * 64 * R + r * 64 + lane;
      tk.offer(md[s], mp[s]);
    }
  const int k = a.k;
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int s = r * 64 + lane;
    const bool valid = (s < k) && (tk.p[r] != kNoPos);
    count += (uint32_t)__popcll(__ballot(valid));
    if (s < k) {
      a.out_ids[q * k + s] = valid ? a.ids[tk.p[r]] : ~0ull;
      a.out_dists[q * k + s] = valid ? tk.d[r] : f_inf();
      if (a.out_pos) a.out_pos[q * k + s] = valid ? tk.p[r] : kNoPos;
    }
  }
  if (lane == 0) a.out_counts[q] = count;
}

using ScanFn = void (*)(IvfPqScanArgs, int);

// Launch shape per specialisation: threads, code vectors in flight per lane,
// and lists per LUT group (G LUTs of M KiB each stay within 64 KiB of LDS so
// two 512-thread workgroups fit a CU's 160 KiB).
template <int MT, int DT>
struct ScanShape {
  static constexpr int NT = 256, U = 1, GMAX = 8;
};
template <>
struct ScanShape<16, 8> {
#ifndef FDB_SCAN168_SHAPE
  // measured on the 1M x 128 / nprobe 16 workload against NT 256-1024,
  // U 1-8, G 1-4: two 16 KiB tables per group keeps 3 workgroups per CU
  static constexpr int NT = 512, U = 2, GMAX = 2;
#else
  static constexpr int NT = FDB_SCAN168_NT, U = FDB_SCAN168_U, GMAX = FDB_SCAN168_G;
#endif
};
template <>
struct ScanShape<32, 3> {
  static constexpr int NT = 512, U = 2, GMAX = 2;
};

template <int MT, int DT, int ORDER, int FAST>
ScanFn pick_scan_r(int R) {
  using S = ScanShape<MT, DT>;
  // k above 256 needs 8-16 top-k registers per list: one batch in flight
  switch (R) {
    case 1: return ivfpq_scan_kernel<MT, DT, 1, ORDER, S::NT, S::U, S::GMAX, FAST>;
    case 2: return ivfpq_scan_kernel<MT, DT, 2, ORDER, S::NT, S::U, S::GMAX, FAST>;
    case 4: return ivfpq_scan_kernel<MT, DT, 4, ORDER, S::NT, S::U, S::GMAX, FAST>;
    case 8: return ivfpq_scan_kernel<MT, DT, 8, ORDER, S::NT, 1, S::GMAX, FAST>;
    case 16: return ivfpq_scan_kernel<MT, DT, 16, ORDER, S::NT, 1, S::GMAX, FAST>;
  }
  return nullptr;
}

// The fast LUT does not reproduce the reference's rounding, so its summation
// order is immaterial: it always uses the 8-lane order.
template <int MT, int DT>
ScanFn pick_scan(int R, int order, int fast) {
  if constexpr (MT > 0) {
    if (fast) return pick_scan_r<MT, DT, kAdcLanes8, 1>(R);
  } else {
    if (fast) return nullptr;
  }
  return order == kAdcLanes8 ? pick_scan_r<MT, DT, kAdcLanes8, 0>(R)
                             : pick_scan_r<MT, DT, kAdcGroups4, 0>(R);
}

int topk_regs(int k) {
  int r = (k + 63) / 64;
  int p = 1;
  while (p < r) p <<= 1;
  return p;
}

// ---------------------------------------------------------------------------
// Build side.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void transpose_centroids_kernel(const float* __restrict__ cents,
                                                                       int k, int dim,
                                                                       float* __restrict__ centT) {
  const int ldc = centT_ld(k);
  const uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= (uint64_t)ldc * dim) return;
  const int c = (int)(e / dim);
  const int d = (int)(e - (uint64_t)c * dim);
  const int d8 = dim / 8;
  const int row = (d >= 8 * d8) ? d : (d % 8) * d8 + d / 8;
  centT[(uint64_t)row * ldc + c] = (c < k) ? cents[e] : 0.0f;
}

// One workgroup per cluster; thread t owns dimensions t, t+256, ...; the
// members are added in ascending point order, as the reference's sequential
// loop over points does.
__global__ __launch_bounds__(kThreads) void kmeans_update_kernel(
    const float* __restrict__ points, int dim, const uint32_t* __restrict__ members,
    const uint32_t* __restrict__ member_off, const float* __restrict__ old_cents,
    float* __restrict__ new_cents) {
  const int c = blockIdx.x;
  const uint32_t s = member_off[c], e = member_off[c + 1];
  for (int d = threadIdx.x; d < dim; d += kThreads) {
    float out;
    if (s == e) {
      out = old_cents[(uint64_t)c * dim + d];
    } else {
      float sum = 0.0f;
      for (uint32_t i = s; i < e; ++i) sum = sum + points[(uint64_t)members[i] * dim + d];
      out = sum / (float)(e - s);
    }
    new_cents[(uint64_t)c * dim + d] = out;
  }
}

// Thread per (row, subspace): argmin over the 256 codewords with the first
// minimum kept (min_by), distances in the reference order on the residual
// r = x - c computed in f32.
template <int DT>
__global__ __launch_bounds__(kThreads) void pq_encode_kernel(
    const float* __restrict__ vectors, const uint64_t* __restrict__ rows,
    const int32_t* __restrict__ row_list, uint64_t n, int dim, const float* __restrict__ centroids,
    const float* __restrict__ codebooks, int M, int dsub_rt, uint8_t* __restrict__ codes) {
  const int dsub = DT ? DT : dsub_rt;
  const uint64_t e = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  if (e >= n * (uint64_t)M) return;
  const uint64_t p = e / M;
  const int m = (int)(e - p * M);
  const float* __restrict__ x = vectors + rows[p] * (uint64_t)dim + (uint64_t)m * dsub;
  const float* __restrict__ c = centroids + (uint64_t)row_list[p] * dim + (uint64_t)m * dsub;
  const float* __restrict__ cb = codebooks + (uint64_t)m * 256 * dsub;
  float best;
  int bi = 0;
  if constexpr (DT > 0) {
    float r[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) r[t] = x[t] - c[t];
    best = l2sq_ref<DT>(r, cb);
    for (int j = 1; j < 256; ++j) {
      const float d = l2sq_ref<DT>(r, cb + j * DT);
      if (best > d) {
        best = d;
        bi = j;
      }
    }
  } else {
    // residual recomputed per codeword; x[t] - c[t] rounds identically each time
    auto dist_to = [&](int j) {
      const float* b = cb + (uint64_t)j * dsub;
      const int nb = dsub / 8;
      float total = 0.0f;
      if (nb > 0) {
        float lane[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) lane[l] = 0.0f;
        for (int i = 0; i < nb; ++i)
#pragma unroll
          for (int l = 0; l < 8; ++l) {
            const float df = (x[8 * i + l] - c[8 * i + l]) - b[8 * i + l];
            lane[l] = __builtin_fmaf(df, df, lane[l]);
          }
        total = lane[0];
#pragma unroll
        for (int l = 1; l < 8; ++l) total = total + lane[l];
      }
      for (int i = 8 * nb; i < dsub; ++i) {
        const float df = (x[i] - c[i]) - b[i];
        total = total + df * df;
      }
      return total;
    };
    best = dist_to(0);
    for (int j = 1; j < 256; ++j) {
      const float d = dist_to(j);
      if (best > d) {
        best = d;
        bi = j;
      }
    }
  }
  codes[p * M + m] = (uint8_t)bi;
}

}  // namespace

int coarse_parts(uint64_t nq, int nlist, int nsel) {
  const uint64_t tiles = (nq + kCoarseQB - 1) / kCoarseQB;
  const int sweeps = centT_ld(nlist) / 256;
  if (nq == 0 || tiles >= kCoarseTargetWG || sweeps < 2) return 1;
  int parts = (int)std::min<uint64_t>((kCoarseTargetWG + tiles - 1) / tiles, (uint64_t)sweeps);
  // every part must still hold nsel centroids
  parts = std::min(parts, std::max(1, nlist / std::max(nsel, 1)));
  while (parts > 1 && nq * (uint64_t)parts * nsel > kCoarsePartEntries) --parts;
  if (parts <= 1) return 1;
  // equal whole sweeps per part, none empty
  const int per = (sweeps + parts - 1) / parts;
  return (sweeps + per - 1) / per;
}

hipError_t launch_coarse_select(const float* queries, uint64_t nq, int dim, const float* centT,
                                int nlist, int nsel, int32_t* out_lists, float* out_dists,
                                int* err_flag, hipStream_t stream, float* part_d,
                                uint32_t* part_k, uint64_t part_cap, const int* only) {
  if (nq == 0) return hipSuccess;
  if (nsel <= 0 || nsel > 1024 || nlist <= 0 || dim <= 0 || dim > 2048) return hipErrorInvalidValue;
  int parts = (part_d && part_k && !only) ? coarse_parts(nq, nlist, nsel) : 1;
  if (parts > 1 && nq * (uint64_t)parts * nsel > part_cap) return hipErrorInvalidValue;
  const int ld = centT_ld(nlist);
#define FDB_CS(R)                                                                                  \
  return launch_coarse_t<R>(queries, nq, dim, centT, ld, nlist, nsel, out_lists, out_dists, err_flag, \
                            parts, part_d, part_k, only, stream);
  switch (topk_regs(nsel)) {
    case 1: FDB_CS(1)
    case 2: FDB_CS(2)
    case 4: FDB_CS(4)
    case 8: FDB_CS(8)
    case 16: FDB_CS(16)
  }
#undef FDB_CS
  return hipErrorInvalidValue;
}

hipError_t launch_ivfpq_scan(const IvfPqScanArgs& a, hipStream_t stream) {
  if (a.nq == 0) return hipSuccess;
  if (a.k <= 0 || a.k > 1024 || a.M <= 0 || a.dsub <= 0) return hipErrorInvalidValue;
  const int R = topk_regs(a.k);
  ScanFn fn;
  int G, nt;
  bool static_lds = true;  // specialised shapes size their LDS at compile time
  if (a.M == 16 && a.dsub == 8) {
    fn = pick_scan<16, 8>(R, a.order, a.lut_mode);
    G = ScanShape<16, 8>::GMAX;
    nt = ScanShape<16, 8>::NT;
  } else if (a.M == 32 && a.dsub == 3) {
    fn = pick_scan<32, 3>(R, a.order, a.lut_mode);
    G = ScanShape<32, 3>::GMAX;
    nt = ScanShape<32, 3>::NT;
  } else {
    fn = pick_scan<0, 0>(R, a.order, a.lut_mode);
    G = std::max(1, std::min(ScanShape<0, 0>::GMAX, 64 / a.M));
    nt = ScanShape<0, 0>::NT;
    static_lds = false;
  }
  if (!fn) return hipErrorInvalidValue;
  const size_t lut_bytes = sizeof(float) * ((size_t)G * a.M * 256 + (size_t)G * a.dim);
  const size_t merge_bytes = (size_t)(nt / 64) * 64 * R * 8;
  if (std::max(lut_bytes, merge_bytes) > 160 * 1024) return hipErrorInvalidValue;
  const size_t lds = static_lds ? 0 : std::max(lut_bytes, merge_bytes);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void*)fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)lds);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3((unsigned)a.nq), dim3(nt), lds, stream, a, G);
  return hipGetLastError();
}

namespace {
__global__ __launch_bounds__(kThreads) void codebook_norms_kernel(const float* __restrict__ cb, int n,
                                                                  int dsub, float* __restrict__ out) {
  const int e = blockIdx.x * kThreads + threadIdx.x;
  if (e >= n) return;
  float s = 0.0f;
  for (int t = 0; t < dsub; ++t) s = __builtin_fmaf(cb[(uint64_t)e * dsub + t], cb[(uint64_t)e * dsub + t], s);
  out[e] = s;
}
}  // namespace

namespace {
// One thread per bitmap word: 32 positions, each id looked up by binary
// search in the sorted allowed list.
__global__ __launch_bounds__(256) void filter_bitmap_kernel(const uint64_t* __restrict__ ids, uint64_t n,
                                                            const uint64_t* __restrict__ allowed,
                                                            uint64_t n_allowed,
                                                            const uint32_t* __restrict__ live,
                                                            uint32_t* __restrict__ out) {
  const uint64_t w = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (w >= (n + 31) / 32) return;
  uint32_t word = 0;
  for (int b = 0; b < 32; ++b) {
    const uint64_t p = w * 32 + b;
    if (p >= n) break;
    if (live && !((live[w] >> b) & 1u)) continue;
    const uint64_t id = ids[p];
    uint64_t lo = 0, hi = n_allowed;  // first allowed entry >= id
    while (lo < hi) {
      const uint64_t mid = (lo + hi) >> 1;
      if (allowed[mid] < id) lo = mid + 1; else hi = mid;
    }
    if (lo < n_allowed && allowed[lo] == id) word |= 1u << b;
  }
  out[w] = word;
}
}  // namespace

hipError_t launch_filter_bitmap(const uint64_t* ids, uint64_t n, const uint64_t* allowed,
                                uint64_t n_allowed, const uint32_t* live, uint32_t* out,
                                hipStream_t stream) {
  const uint64_t words = (n + 31) / 32;
  if (words == 0) return hipSuccess;
  hipLaunchKernelGGL(filter_bitmap_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                     ids, n, allowed, n_allowed, live, out);
  return hipGetLastError();
}

hipError_t launch_codebook_norms(const float* codebooks, int M, int dsub, float* out,
                                 hipStream_t stream) {
  const int n = M * 256;
  hipLaunchKernelGGL(codebook_norms_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0,
                     stream, codebooks, n, dsub, out);
  return hipGetLastError();
}

hipError_t launch_kmeans_update(const float* points, int dim, const uint32_t* members,
                                const uint32_t* member_off, int k, const float* old_cents,
                                float* new_cents, hipStream_t stream) {
  if (k <= 0) return hipSuccess;
  hipLaunchKernelGGL(kmeans_update_kernel, dim3(k), dim3(kThreads), 0, stream, points, dim, members,
                     member_off, old_cents, new_cents);
  return hipGetLastError();
}

hipError_t launch_pq_encode(const float* vectors, const uint64_t* rows, const int32_t* row_list,
                            uint64_t n, int dim, const float* centroids, const float* codebooks,
                            int M, int dsub, uint8_t* codes, hipStream_t stream) {
  const uint64_t total = n * (uint64_t)M;
  if (total == 0) return hipSuccess;
  const unsigned blocks = (unsigned)((total + kThreads - 1) / kThreads);
  switch (dsub) {
    case 8:
      hipLaunchKernelGGL(pq_encode_kernel<8>, dim3(blocks), dim3(kThreads), 0, stream, vectors, rows,
                         row_list, n, dim, centroids, codebooks, M, dsub, codes);
      break;
    case 3:
      hipLaunchKernelGGL(pq_encode_kernel<3>, dim3(blocks), dim3(kThreads), 0, stream, vectors, rows,
                         row_list, n, dim, centroids, codebooks, M, dsub, codes);
      break;
    case 4:
      hipLaunchKernelGGL(pq_encode_kernel<4>, dim3(blocks), dim3(kThreads), 0, stream, vectors, rows,
                         row_list, n, dim, centroids, codebooks, M, dsub, codes);
      break;
    default:
      hipLaunchKernelGGL(pq_encode_kernel<0>, dim3(blocks), dim3(kThreads), 0, stream, vectors, rows,
                         row_list, n, dim, centroids, codebooks, M, dsub, codes);
  }
  return hipGetLastError();
}

hipError_t launch_transpose_centroids(const float* cents, int k, int dim, float* centT,
                                      hipStream_t stream) {
  const uint64_t total = (uint64_t)centT_ld(k) * dim;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(transpose_centroids_kernel, dim3((unsigned)((total + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, cents, k, dim, centT);
  return hipGetLastError();
}

}  // namespace fdb
