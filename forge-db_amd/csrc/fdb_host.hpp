// Host-side helpers: error propagation, device buffers, and the scalar
// reference-order distance used by host-side training steps.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "forgedb_hip.h"

namespace fdb {

struct Error : std::runtime_error {
  int status;
  Error(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};

void set_last_error(const std::string& msg);

inline void hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  (void)hipGetLastError();  // clear the sticky launch error
  const int st = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? FDB_ERR_OUT_OF_MEMORY
                                                                             : FDB_ERR_HIP;
  throw Error(st, std::string(what) + ": " + hipGetErrorString(e));
}
#define FDB_HIP(expr) ::fdb::hip_check((expr), #expr)

template <class T>
struct DevBuf {
  T* p = nullptr;
  size_t n = 0;
  DevBuf() = default;
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  ~DevBuf() { release(); }
  void release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
  }
  // (re)allocate to hold at least cnt elements; contents are not kept
  void reserve(size_t cnt) {
    if (cnt <= n && p) return;
    release();
    if (cnt == 0) return;
    FDB_HIP(hipMalloc((void**)&p, cnt * sizeof(T)));
    n = cnt;
  }
  void upload(const T* src, size_t cnt, hipStream_t s) {
    reserve(cnt);
    if (cnt) FDB_HIP(hipMemcpyAsync(p, src, cnt * sizeof(T), hipMemcpyHostToDevice, s));
  }
};

// Orders a handle's device work across streams.  Every call shares the
// handle's device scratch, so a call enqueued on stream s first makes s wait
// (on the GPU) for the work the previous call enqueued, when that call used
// another stream; same-stream calls are ordered by the stream already.
// Used under the handle's mutex, through OrderedOn.
struct StreamOrder {
  hipEvent_t ev = nullptr;
  hipStream_t last = nullptr;
  bool pending = false;
  StreamOrder() = default;
  StreamOrder(const StreamOrder&) = delete;
  StreamOrder& operator=(const StreamOrder&) = delete;
  ~StreamOrder() {
    if (ev) (void)hipEventDestroy(ev);
  }
  // creates the event (a handle's constructor calls this, so that calls
  // need not)
  void init() {
    if (!ev) FDB_HIP(hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  }
  void begin(hipStream_t s) {
    if (pending && last != s) FDB_HIP(hipStreamWaitEvent(s, ev, 0));
  }
  // the host waits for the previous call's work
  void wait_host() {
    if (pending) FDB_HIP(hipEventSynchronize(ev));
  }
  // no throw: runs from a destructor, also after a failed call
  void end(hipStream_t s) noexcept {
    if (!ev && hipEventCreateWithFlags(&ev, hipEventDisableTiming) != hipSuccess) {
      ev = nullptr;
      return;
    }
    if (hipEventRecord(ev, s) == hipSuccess) {
      last = s;
      pending = true;
    }
  }
};

// The scope of one call's device work on stream s.
struct OrderedOn {
  StreamOrder& o;
  hipStream_t s;
  OrderedOn(StreamOrder& order, hipStream_t stream) : o(order), s(stream) { o.begin(s); }
  ~OrderedOn() { o.end(s); }
  OrderedOn(const OrderedOn&) = delete;
  OrderedOn& operator=(const OrderedOn&) = delete;
};

// Coefficients of the fp16 screening bound |s - d| <= c_dot |r| X' +
// c_sq (|r| + X')^2, X' = X + cabs, for s = |r|^2 + |x|^2 - 2<r^, x^> with
// r^, x^ the operands scaled into [2^12, 2^13) and rounded to fp16, the
// product accumulated in fp32 on the matrix cores, against a reference
// value d that is a sum of non-negative terms each rounded at most n_ref
// times.  With u = 2^-24, uh = 2^-11 and D16 the padded dimension:
//   each converted component is within uh relative plus 2^-26 of the
//   operand's largest component (flushed fp16 subnormals included), so
//   <r^, x^> (unscaled) is within h' |r| X' of <r, x>, where
//   h' = 2uh + uh^2 + 2.002 * 2^-26 sqrt(D16) + 1.002 g2,
//   g2 = 2u D16 / (1 - 2u D16) covering fp32 accumulation in any order
//   (rounded or truncated), and X' = X + 2^-26 sqrt(D16) cmax for rows of
//   norm <= X and largest component cmax;
//   |r|^2 and |x|^2 in fp32 are within gamma_D16 (|r| + X)^2 together, the
//   final add and FMA within 3u (|r| + X')^2, and the reference's rounding
//   within gamma_(n_ref) d <= gamma_(n_ref) (|r| + X)^2.
// Everything gets a 1.1 slack factor.
inline void screen_eps_coeffs(int D16, int n_ref, float cmax, float& c_dot, float& c_sq, float& cabs) {
  const double u = std::ldexp(1.0, -24), uh = std::ldexp(1.0, -11);
  const double g2 = 2.0 * u * D16 / (1.0 - 2.0 * u * D16);
  const double hp = 2.0 * uh + uh * uh + 2.002 * std::ldexp(1.0, -26) * std::sqrt((double)D16) + 1.002 * g2 +
                    D16 * std::ldexp(1.0, -52);
  const double gD = D16 * u / (1.0 - D16 * u);
  const double ga = n_ref * u / (1.0 - n_ref * u);
  c_dot = (float)(1.1 * 2.0 * hp);
  c_sq = (float)(1.1 * (gD + 3.0 * u + ga));
  cabs = (float)(1.0001 * std::ldexp(1.0, -26) * std::sqrt((double)D16) * cmax);
}

// Squared L2 in the reference's AVX2 order (src/distance/simd.rs:335-366),
// scalar: 8 FMA lanes, lanes summed from -0.0 left to right, scalar tail.
inline float host_l2sq_ref(const float* a, const float* b, int n) {
  const int nb = n / 8;
  float lane[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = 0; i < nb; ++i)
    for (int l = 0; l < 8; ++l) {
      const float d = a[8 * i + l] - b[8 * i + l];
      lane[l] = std::fma(d, d, lane[l]);
    }
  float total = -0.0f;
  for (int l = 0; l < 8; ++l) total += lane[l];
  for (int i = 8 * nb; i < n; ++i) {
    const float d = a[i] - b[i];
    total += d * d;
  }
  return total;
}

// SplitMix64: the i-th output for a seed is a pure function of (seed, i).
inline uint64_t splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

struct Stream {
  uint64_t seed, n = 0;
  explicit Stream(uint64_t s) : seed(s) {}
  uint64_t next() { return splitmix64_at(seed, n++); }
  uint64_t index(uint64_t bound) { return (uint64_t)(((unsigned __int128)next() * bound) >> 64); }
  float unit() { return (float)(next() >> 40) * (1.0f / 16777216.0f); }
};

// Fisher-Yates from the back (rand 0.8 SliceRandom::shuffle).
inline void shuffle(Stream& rng, std::vector<uint64_t>& v) {
  for (uint64_t i = v.size(); i > 1; --i) {
    const uint64_t j = rng.index(i);
    std::swap(v[i - 1], v[j]);
  }
}

}  // namespace fdb
