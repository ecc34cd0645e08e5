// Device-side building blocks shared by the forge-db HIP kernels (gfx950,
// wave64).  Everything here is compiled with -ffp-contract=off: a product
// written as `a * b + c` stays a rounded multiply and a rounded add, and the
// only fused operations are the explicit __builtin_fmaf calls, placed where
// the reference's AVX2 kernels issue _mm256_fmadd_ps.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdb {

constexpr int kWave = 64;
constexpr uint32_t kNoPos = 0xFFFFFFFFu;

__device__ __forceinline__ float f_inf() { return __builtin_huge_valf(); }

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}
__device__ __forceinline__ uint32_t readlane_u(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}

// ---------------------------------------------------------------------------
// Squared L2 in the reference's AVX2 order (src/distance/simd.rs:335-366):
// lane l = FMA chain over elements i = l (mod 8) of the full 8-blocks, lanes
// summed left to right, then the tail i >= 8*floor(n/8) as `total += d*d`
// (separate multiply and add).  `a` is read element by element, so it may
// live in LDS (wave-uniform reads broadcast).
// ---------------------------------------------------------------------------
template <int N>
__device__ __forceinline__ float l2sq_ref(const float* __restrict__ a, const float* __restrict__ b) {
  constexpr int NB = N / 8;
  float total;
  if constexpr (NB > 0) {
    float lane[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) {
      float d = a[l] - b[l];
      lane[l] = __builtin_fmaf(d, d, 0.0f);
    }
#pragma unroll
    for (int i = 1; i < NB; ++i)
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        float d = a[8 * i + l] - b[8 * i + l];
        lane[l] = __builtin_fmaf(d, d, lane[l]);
      }
    total = lane[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) total = total + lane[l];
  } else {
    total = 0.0f;
  }
#pragma unroll
  for (int i = 8 * NB; i < N; ++i) {
    float d = a[i] - b[i];
    total = total + d * d;
  }
  return total;
}

// Same order for a runtime length.
__device__ __forceinline__ float l2sq_ref_rt(const float* __restrict__ a, const float* __restrict__ b,
                                             int n) {
  const int nb = n / 8;
  float total = 0.0f;
  if (nb > 0) {
    float lane[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) lane[l] = 0.0f;
    for (int i = 0; i < nb; ++i)
#pragma unroll
      for (int l = 0; l < 8; ++l) {
        float d = a[8 * i + l] - b[8 * i + l];
        lane[l] = __builtin_fmaf(d, d, lane[l]);
      }
    total = lane[0];
#pragma unroll
    for (int l = 1; l < 8; ++l) total = total + lane[l];
  }
  for (int i = 8 * nb; i < n; ++i) {
    float d = a[i] - b[i];
    total = total + d * d;
  }
  return total;
}

// ---------------------------------------------------------------------------
// ADC summation orders over a flat LUT [M][256] (src/pq.rs).
// ---------------------------------------------------------------------------
enum AdcOrder : int {
  kAdcLanes8 = 0,   // asymmetric_distance_simd_avx2 / batch_..._avx2, pq.rs:318-485
  kAdcGroups4 = 1,  // asymmetric_distance_fast, pq.rs:218-245
};

template <int M>
__device__ __forceinline__ uint32_t code_byte(const uint32_t (&w)[(M + 3) / 4], int m) {
  return (w[m >> 2] >> (8 * (m & 3))) & 0xFFu;
}

template <int M, int ORDER>
__device__ __forceinline__ float adc_sum(const float* __restrict__ lut, const uint32_t (&w)[(M + 3) / 4]) {
  if constexpr (ORDER == kAdcLanes8) {
    constexpr int MB = M / 8;
    float total;
    if constexpr (MB > 0) {
      float lane[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) lane[l] = lut[l * 256 + code_byte<M>(w, l)];
#pragma unroll
      for (int b = 1; b < MB; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) lane[l] = lane[l] + lut[(8 * b + l) * 256 + code_byte<M>(w, 8 * b + l)];
      total = lane[0];
#pragma unroll
      for (int l = 1; l < 8; ++l) total = total + lane[l];
    } else {
      total = 0.0f;
    }
#pragma unroll
    for (int m = 8 * MB; m < M; ++m) total = total + lut[m * 256 + code_byte<M>(w, m)];
    return total;
  } else {
    float sum = 0.0f;
    constexpr int MG = M / 4;
#pragma unroll
    for (int g = 0; g < MG; ++g) {
      float t = lut[(4 * g) * 256 + code_byte<M>(w, 4 * g)] +
                lut[(4 * g + 1) * 256 + code_byte<M>(w, 4 * g + 1)];
      t = t + lut[(4 * g + 2) * 256 + code_byte<M>(w, 4 * g + 2)];
      t = t + lut[(4 * g + 3) * 256 + code_byte<M>(w, 4 * g + 3)];
      sum = sum + t;
    }
#pragma unroll
    for (int m = 4 * MG; m < M; ++m) sum = sum + lut[m * 256 + code_byte<M>(w, m)];
    return sum;
  }
}

// Runtime-M versions reading bytes directly.
template <int ORDER>
__device__ __forceinline__ float adc_sum_rt(const float* __restrict__ lut, const uint8_t* __restrict__ c,
                                            int M) {
  if (ORDER == kAdcLanes8) {
    const int mb = M / 8;
    float total = 0.0f;
    if (mb > 0) {
      float lane[8];
#pragma unroll
      for (int l = 0; l < 8; ++l) lane[l] = lut[l * 256 + c[l]];
      for (int b = 1; b < mb; ++b)
#pragma unroll
        for (int l = 0; l < 8; ++l) lane[l] = lane[l] + lut[(8 * b + l) * 256 + c[8 * b + l]];
      total = lane[0];
#pragma unroll
      for (int l = 1; l < 8; ++l) total = total + lane[l];
    }
    for (int m = 8 * mb; m < M; ++m) total = total + lut[m * 256 + c[m]];
    return total;
  } else {
    float sum = 0.0f;
    int m = 0;
    for (; m + 4 <= M; m += 4) {
      float t = lut[m * 256 + c[m]] + lut[(m + 1) * 256 + c[m + 1]];
      t = t + lut[(m + 2) * 256 + c[m + 2]];
      t = t + lut[(m + 3) * 256 + c[m + 3]];
      sum = sum + t;
    }
    for (; m < M; ++m) sum = sum + lut[m * 256 + c[m]];
    return sum;
  }
}

// ---------------------------------------------------------------------------
// Wave64 top-k.  One sorted list of 64*R (distance, key) pairs spread over
// the wave: slot s = r*64 + lane lives in register r of that lane.  Pairs are
// ordered by distance, then by key (a list position, centroid index or
// candidate rank), so the k smallest are the same set whatever order they are
// offered in; exact distance ties resolve to the smaller key.  The reference
// leaves that order to BinaryHeap / select_nth_unstable, so this is one of
// the orders it can produce.  An empty slot is (+inf, kNoPos), which no
// offered pair with key kNoPos can displace.
// ---------------------------------------------------------------------------
__device__ __forceinline__ bool pair_lt(float d1, uint32_t p1, float d2, uint32_t p2) {
  return d1 < d2 || (d1 == d2 && p1 < p2);
}

template <int R>
struct WaveTopK {
  float d[R];
  uint32_t p[R];
  float tau;      // pair in slot k-1 (wave-uniform); (+inf, kNoPos) until k arrived
  uint32_t tau_p;
  int k;

  __device__ __forceinline__ void init(int kk) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      d[r] = f_inf();
      p[r] = kNoPos;
    }
    k = kk;
    tau = f_inf();
    tau_p = kNoPos;
  }

  __device__ __forceinline__ void read_tau() {
    const int s = k - 1;
    const int rs = s >> 6;
    // running comparison, not `r == rs`: an equality select chain over an
    // array is turned into an indexed (scratch) access by the compiler
    float v = d[0];
    uint32_t w = p[0];
#pragma unroll
    for (int r = 1; r < R; ++r) {
      const bool in = r <= rs;
      v = in ? d[r] : v;
      w = in ? p[r] : w;
    }
    tau = readlane_f(v, s & 63);
    tau_p = readlane_u(w, s & 63);
  }

  // Insert one wave-uniform pair.  Caller guarantees (dn, pn) < (tau, tau_p).
  __device__ __forceinline__ void insert(float dn, uint32_t pn) {
    const int lane = lane_id();
    int pos = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) pos += __popcll(__ballot(pair_lt(d[r], p[r], dn, pn)));
#pragma unroll
    for (int r = R - 1; r >= 0; --r) {
      float up_d = __shfl_up(d[r], 1);
      uint32_t up_p = __shfl_up(p[r], 1);
      if (r > 0) {
        float cd = readlane_f(d[r - 1], 63);
        uint32_t cp = readlane_u(p[r - 1], 63);
        if (lane == 0) {
          up_d = cd;
          up_p = cp;
        }
      }
      const int s = r * 64 + lane;
      if (s > pos) {
        d[r] = up_d;
        p[r] = up_p;
      } else if (s == pos) {
        d[r] = dn;
        p[r] = pn;
      }
    }
    read_tau();
  }

  // Every lane offers one pair; a lane with nothing to offer passes
  // (+inf, kNoPos).
  __device__ __forceinline__ void offer(float dist, uint32_t key) {
    uint64_t mask = __ballot(pair_lt(dist, key, tau, tau_p));
    drain(mask, dist, key);
  }

  // Hot-loop form: `valid` lanes offer (dist, key).  The per-lane test is a
  // single compare (dist <= tau); the exact pair order is checked only for
  // the few lanes that pass it.
  __device__ __forceinline__ void offer_valid(float dist, uint32_t key, bool valid) {
    uint64_t mask = __ballot(valid && dist <= tau);
    drain(mask, dist, key);
  }

  // Lanes in mask bring a pair that may enter the list.  A few are inserted
  // one at a time; many (an empty list filling up) are merged in bulk.
  __device__ __forceinline__ void drain(uint64_t mask, float dist, uint32_t key) {
    if (__popcll(mask) > kBulkThreshold) {
      const bool in = (mask >> lane_id()) & 1;
      merge64(in ? dist : f_inf(), in ? key : kNoPos);
      return;
    }
    while (mask) {
      const int l = __ffsll((unsigned long long)mask) - 1;
      mask &= mask - 1;
      const float dn = readlane_f(dist, l);
      const uint32_t pn = readlane_u(key, l);
      if (pair_lt(dn, pn, tau, tau_p)) insert(dn, pn);
    }
  }

  static constexpr int kBulkThreshold = 6;

  // Queued form of offer_valid for long scans.  Lanes that pass the
  // threshold append their pair to a wave-private LDS queue q of 64 slots
  // (qn pairs held, wave-uniform); a queue that would overflow is merged
  // into the list in one merge64.  The threshold only moves at a merge, so a
  // queued pair may turn out not to belong: the merge keeps the 64*R
  // smallest of list and queue whatever was let in.  Call flush() before
  // reading the list.
  __device__ __forceinline__ void offer_queued(float dist, uint32_t key, bool valid, uint2* q, int& qn) {
    uint64_t mask = __ballot(valid && dist <= tau);
    if (mask == 0) return;
    if (qn + __popcll(mask) > 64) {
      flush(q, qn);
      mask = __ballot(valid && dist <= tau);
    }
    const uint32_t before = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                      __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
    if ((mask >> lane_id()) & 1) q[qn + (int)before] = make_uint2(__float_as_uint(dist), key);
    qn += __popcll(mask);
  }

  // Merges the queue (qn pairs) into the list and empties it.  Queue slots
  // are written and read by different lanes of the one wave; LDS operations
  // of a wave complete in issue order, and the wave barriers keep the
  // compiler from moving them across each other.
  __device__ __forceinline__ void flush(uint2* q, int& qn) {
    if (qn == 0) return;
    __builtin_amdgcn_wave_barrier();
    const int lane = lane_id();
    const uint2 e = lane < qn ? q[lane] : make_uint2(__float_as_uint(f_inf()), kNoPos);
    __builtin_amdgcn_wave_barrier();
    merge64(__uint_as_float(e.x), e.y);
    qn = 0;
  }

  // One compare-exchange of a bitonic network: keep the smaller pair when
  // keep_min, else the larger.
  static __device__ __forceinline__ void cx(float& d0, uint32_t& p0, float d1, uint32_t p1,
                                            bool keep_min) {
    const bool other_first = pair_lt(d1, p1, d0, p0);
    if (other_first == keep_min) {
      d0 = d1;
      p0 = p1;
    }
  }

  // Merge one pair per lane (sentinel (+inf, kNoPos) for none) into the
  // list: sort the 64 new pairs (bitonic network over the lanes), reverse
  // them against the list's last register so list-then-reversed is bitonic,
  // keep the smaller of each position (the 64*R smallest of both, still
  // bitonic), then sort that bitonic sequence.
  __device__ __forceinline__ void merge64(float nd, uint32_t np) {
    const int lane = lane_id();
#pragma unroll
    for (int kk = 2; kk <= 64; kk <<= 1) {
#pragma unroll
      for (int j = kk >> 1; j > 0; j >>= 1) {
        const float od = __shfl_xor(nd, j);
        const uint32_t op = __shfl_xor(np, j);
        const bool lower = (lane & j) == 0;
        const bool up = (lane & kk) == 0;
        cx(nd, np, od, op, lower == up);
      }
    }
    const float rd = __shfl(nd, 63 - lane);
    const uint32_t rp = __shfl(np, 63 - lane);
    cx(d[R - 1], p[R - 1], rd, rp, true);
#pragma unroll
    for (int dist = 32 * R; dist >= 64; dist >>= 1) {
      const int rs = dist / 64;
#pragma unroll
      for (int r = 0; r < R; ++r)
        if ((r & rs) == 0) {
          float lo_d = d[r], hi_d = d[r + rs];
          uint32_t lo_p = p[r], hi_p = p[r + rs];
          const bool swap = pair_lt(hi_d, hi_p, lo_d, lo_p);
          d[r] = swap ? hi_d : lo_d;
          p[r] = swap ? hi_p : lo_p;
          d[r + rs] = swap ? lo_d : hi_d;
          p[r + rs] = swap ? lo_p : hi_p;
        }
    }
#pragma unroll
    for (int j = 32; j > 0; j >>= 1) {
      const bool lower = (lane & j) == 0;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const float od = __shfl_xor(d[r], j);
        const uint32_t op = __shfl_xor(p[r], j);
        cx(d[r], p[r], od, op, lower);
      }
    }
    read_tau();
  }
};

}  // namespace fdb
