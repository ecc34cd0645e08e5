// refcpu.cpp — CPU restatement of forge-db's query path.  TEST INFRASTRUCTURE:
// this is the oracle and the CPU baseline, never part of the shipped library.
// Built with -O3 -mavx2 -mfma -ffp-contract=off (see oracle/Makefile): the
// last flag keeps every scalar `a*b + c` as a separate multiply and add, as
// Rust compiles it, so only the explicit _mm256_fmadd_ps calls fuse.
#include "refcpu.h"

#include <immintrin.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <queue>
#include <thread>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

// Rust's `impl Sum for f32` folds from -0.0 (it only matters when every term
// is a zero).  Lane arrays are summed left to right like `iter().sum()`.
inline float rust_sum(const float* v, int n) {
  float s = -0.0f;
  for (int i = 0; i < n; ++i) s += v[i];
  return s;
}

// ---------------------------------------------------------------------------
// Distances, AVX2+FMA path — src/distance/simd.rs:290-517.
// ---------------------------------------------------------------------------

// simd.rs:335-366: 8 FMA lanes over i = l (mod 8), lane sum left to right,
// then the scalar tail as a separate multiply and add.
__attribute__((target("avx2,fma"))) float l2sq_avx2(const float* a, const float* b,
                                                    size_t len) {
  __m256 sum = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 8 <= len) {
    __m256 va = _mm256_loadu_ps(a + i);
    __m256 vb = _mm256_loadu_ps(b + i);
    __m256 diff = _mm256_sub_ps(va, vb);
    sum = _mm256_fmadd_ps(diff, diff, sum);
    i += 8;
  }
  alignas(32) float lanes[8];
  _mm256_store_ps(lanes, sum);
  float total = rust_sum(lanes, 8);
  while (i < len) {
    float diff = a[i] - b[i];
    total += diff * diff;
    ++i;
  }
  return total;
}

// simd.rs:375-417
__attribute__((target("avx2"))) float l1_avx2(const float* a, const float* b, size_t len) {
  __m256 sum = _mm256_setzero_ps();
  const __m256 sign_mask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7FFFFFFF));
  size_t i = 0;
  while (i + 8 <= len) {
    __m256 va = _mm256_loadu_ps(a + i);
    __m256 vb = _mm256_loadu_ps(b + i);
    __m256 diff = _mm256_sub_ps(va, vb);
    __m256 abs_diff = _mm256_and_ps(diff, sign_mask);
    sum = _mm256_add_ps(sum, abs_diff);
    i += 8;
  }
  alignas(32) float lanes[8];
  _mm256_store_ps(lanes, sum);
  float total = rust_sum(lanes, 8);
  while (i < len) {
    total += std::fabs(a[i] - b[i]);
    ++i;
  }
  return total;
}

// simd.rs:424-456
__attribute__((target("avx2,fma"))) float dot_avx2(const float* a, const float* b,
                                                   size_t len) {
  __m256 sum = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 8 <= len) {
    __m256 va = _mm256_loadu_ps(a + i);
    __m256 vb = _mm256_loadu_ps(b + i);
    sum = _mm256_fmadd_ps(va, vb, sum);
    i += 8;
  }
  alignas(32) float lanes[8];
  _mm256_store_ps(lanes, sum);
  float total = rust_sum(lanes, 8);
  while (i < len) {
    total += a[i] * b[i];
    ++i;
  }
  return total;
}

// simd.rs:466-517: three FMA streams; a zero denominator gives 0.
__attribute__((target("avx2,fma"))) float cosine_avx2(const float* a, const float* b,
                                                      size_t len) {
  __m256 dot_sum = _mm256_setzero_ps();
  __m256 na_sum = _mm256_setzero_ps();
  __m256 nb_sum = _mm256_setzero_ps();
  size_t i = 0;
  while (i + 8 <= len) {
    __m256 va = _mm256_loadu_ps(a + i);
    __m256 vb = _mm256_loadu_ps(b + i);
    dot_sum = _mm256_fmadd_ps(va, vb, dot_sum);
    na_sum = _mm256_fmadd_ps(va, va, na_sum);
    nb_sum = _mm256_fmadd_ps(vb, vb, nb_sum);
    i += 8;
  }
  alignas(32) float d8[8], a8[8], b8[8];
  _mm256_store_ps(d8, dot_sum);
  _mm256_store_ps(a8, na_sum);
  _mm256_store_ps(b8, nb_sum);
  float dot = rust_sum(d8, 8), na = rust_sum(a8, 8), nb = rust_sum(b8, 8);
  while (i < len) {
    dot += a[i] * b[i];
    na += a[i] * a[i];
    nb += b[i] * b[i];
    ++i;
  }
  float norm_product = std::sqrt(na * nb);
  if (norm_product == 0.0f) return 0.0f;
  return 1.0f - (dot / norm_product);
}

// ---------------------------------------------------------------------------
// PQ ADC orders — src/pq.rs.
// ---------------------------------------------------------------------------

// asymmetric_distance_simd_avx2, pq.rs:435-485: lane l gathers subvectors
// m = l (mod 8); explicit left-to-right lane sum; scalar tail.
__attribute__((target("avx2"))) float adc_lanes8(const float* table, const uint8_t* codes,
                                                 int n) {
  __m256 sum = _mm256_setzero_ps();
  int i = 0;
  while (i + 8 <= n) {
    __m256i idx = _mm256_set_epi32(
        (i + 7) * 256 + codes[i + 7], (i + 6) * 256 + codes[i + 6],
        (i + 5) * 256 + codes[i + 5], (i + 4) * 256 + codes[i + 4],
        (i + 3) * 256 + codes[i + 3], (i + 2) * 256 + codes[i + 2],
        (i + 1) * 256 + codes[i + 1], i * 256 + codes[i]);
    __m256 v = _mm256_i32gather_ps(table, idx, 4);
    sum = _mm256_add_ps(sum, v);
    i += 8;
  }
  alignas(32) float s[8];
  _mm256_store_ps(s, sum);
  float total = s[0] + s[1] + s[2] + s[3] + s[4] + s[5] + s[6] + s[7];
  while (i < n) {
    total += table[i * 256 + codes[i]];
    ++i;
  }
  return total;
}

// batch_asymmetric_distance_avx2, pq.rs:318-402: 4 queries share the index
// vector; each lane sum folds with iter().sum(); fewer than 4 remaining
// queries fall back to adc_lanes8.
__attribute__((target("avx2"))) void adc_batch(const float* const* tables, int nq,
                                               const uint8_t* codes, int n, float* out) {
  int qi = 0;
  while (qi + 4 <= nq) {
    __m256 s0 = _mm256_setzero_ps(), s1 = _mm256_setzero_ps();
    __m256 s2 = _mm256_setzero_ps(), s3 = _mm256_setzero_ps();
    const float* t0 = tables[qi];
    const float* t1 = tables[qi + 1];
    const float* t2 = tables[qi + 2];
    const float* t3 = tables[qi + 3];
    int m = 0;
    while (m + 8 <= n) {
      __m256i idx = _mm256_set_epi32(
          (m + 7) * 256 + codes[m + 7], (m + 6) * 256 + codes[m + 6],
          (m + 5) * 256 + codes[m + 5], (m + 4) * 256 + codes[m + 4],
          (m + 3) * 256 + codes[m + 3], (m + 2) * 256 + codes[m + 2],
          (m + 1) * 256 + codes[m + 1], m * 256 + codes[m]);
      s0 = _mm256_add_ps(s0, _mm256_i32gather_ps(t0, idx, 4));
      s1 = _mm256_add_ps(s1, _mm256_i32gather_ps(t1, idx, 4));
      s2 = _mm256_add_ps(s2, _mm256_i32gather_ps(t2, idx, 4));
      s3 = _mm256_add_ps(s3, _mm256_i32gather_ps(t3, idx, 4));
      m += 8;
    }
    alignas(32) float a0[8], a1[8], a2[8], a3[8];
    _mm256_store_ps(a0, s0);
    _mm256_store_ps(a1, s1);
    _mm256_store_ps(a2, s2);
    _mm256_store_ps(a3, s3);
    float tot0 = rust_sum(a0, 8), tot1 = rust_sum(a1, 8);
    float tot2 = rust_sum(a2, 8), tot3 = rust_sum(a3, 8);
    while (m < n) {
      int off = m * 256 + codes[m];
      tot0 += t0[off];
      tot1 += t1[off];
      tot2 += t2[off];
      tot3 += t3[off];
      ++m;
    }
    out[qi] = tot0;
    out[qi + 1] = tot1;
    out[qi + 2] = tot2;
    out[qi + 3] = tot3;
    qi += 4;
  }
  while (qi < nq) {
    out[qi] = adc_lanes8(tables[qi], codes, n);
    ++qi;
  }
}

// asymmetric_distance_fast, pq.rs:218-245: groups of 4 summed left to right,
// each group added to the running sum.
float adc_groups4(const float* table, const uint8_t* codes, int n) {
  float sum = 0.0f;
  int i = 0;
  while (i + 4 <= n) {
    sum += table[i * 256 + codes[i]] + table[(i + 1) * 256 + codes[i + 1]] +
           table[(i + 2) * 256 + codes[i + 2]] + table[(i + 3) * 256 + codes[i + 3]];
    i += 4;
  }
  while (i < n) {
    sum += table[i * 256 + codes[i]];
    ++i;
  }
  return sum;
}

// asymmetric_distance_flat_scalar, pq.rs:410-418
float adc_seq(const float* table, const uint8_t* codes, int n) {
  float sum = 0.0f;
  for (int m = 0; m < n; ++m) sum += table[m * 256 + codes[m]];
  return sum;
}

// build_lookup_table_flat, pq.rs:175-189 (build_lookup_table, :149-170, gives
// the same values in nested form).
void pq_lut(const float* cb, int M, int dsub, const float* r, float* lut) {
  for (int m = 0; m < M; ++m)
    for (int j = 0; j < 256; ++j)
      lut[m * 256 + j] = l2sq_avx2(r + (size_t)m * dsub,
                                   cb + ((size_t)m * 256 + j) * dsub, (size_t)dsub);
}

// encode, pq.rs:114-139: min_by keeps the first minimum (a later candidate
// replaces it only when strictly smaller; NaN never replaces).
void pq_encode(const float* cb, int M, int dsub, const float* x, uint8_t* code) {
  for (int m = 0; m < M; ++m) {
    const float* xs = x + (size_t)m * dsub;
    float best = l2sq_avx2(xs, cb + (size_t)m * 256 * dsub, (size_t)dsub);
    int bi = 0;
    for (int j = 1; j < 256; ++j) {
      float d = l2sq_avx2(xs, cb + ((size_t)m * 256 + j) * dsub, (size_t)dsub);
      if (best > d) {
        best = d;
        bi = j;
      }
    }
    code[m] = (uint8_t)bi;
  }
}

// ---------------------------------------------------------------------------
// Thread pool helper: items are claimed in order from an atomic counter, the
// shape of rayon's par_chunks / par_iter for independent items.
// ---------------------------------------------------------------------------
void parallel_for(uint64_t n_items, int nthreads, const std::function<void(uint64_t)>& fn) {
  if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
  if (n_items == 0) return;
  if ((uint64_t)nthreads > n_items) nthreads = (int)n_items;
  if (nthreads == 1) {
    for (uint64_t i = 0; i < n_items; ++i) fn(i);
    return;
  }
  std::atomic<uint64_t> next{0};
  std::vector<std::thread> pool;
  pool.reserve(nthreads);
  for (int t = 0; t < nthreads; ++t)
    pool.emplace_back([&]() {
      for (;;) {
        uint64_t i = next.fetch_add(1);
        if (i >= n_items) break;
        fn(i);
      }
    });
  for (auto& th : pool) th.join();
}

// ---------------------------------------------------------------------------
// Seeded generator.  SplitMix64's i-th output for a seed is a pure function of
// (seed, i), so the stream can be drawn in any order (and vectorised in numpy
// by the data generator).
// ---------------------------------------------------------------------------
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
  // index in [0, bound): multiply-shift on the 64-bit draw
  uint64_t index(uint64_t bound) {
    return (uint64_t)(((unsigned __int128)next() * bound) >> 64);
  }
  // f32 in [0,1) from the top 24 bits
  float unit() { return (float)(next() >> 40) * (1.0f / 16777216.0f); }
};

// rand 0.8 SliceRandom::shuffle: Fisher-Yates from the back.
void shuffle(Stream& rng, std::vector<uint64_t>& v) {
  for (uint64_t i = v.size(); i > 1; --i) {
    uint64_t j = rng.index(i);
    std::swap(v[i - 1], v[j]);
  }
}

// Index of the nearest row by l2sq with min_by's first-minimum rule
// (kmeans.rs:147-160, ivf_pq.rs:403-414).
int nearest(const float* x, const float* cents, int k, int dim) {
  float best = l2sq_avx2(x, cents, (size_t)dim);
  int bi = 0;
  for (int c = 1; c < k; ++c) {
    float d = l2sq_avx2(x, cents + (size_t)c * dim, (size_t)dim);
    if (best > d) {
      best = d;
      bi = c;
    }
  }
  return bi;
}

// KMeans::fit_raw, kmeans.rs:87-193, with the RNG seeded.  Returns 0, or -1
// when n < k (the reference would index past its centroid list).
int kmeans_fit(const float* data, uint64_t n, int dim, int k, int max_iters, uint64_t seed,
               float* out, int nthreads) {
  if (k <= 0 || dim <= 0 || n < (uint64_t)k) return -1;
  Stream rng(seed);
  std::vector<float> cents((size_t)k * dim);
  auto row = [&](uint64_t i) { return data + i * (uint64_t)dim; };
  if (k > 64) {  // KMEANSPP_THRESHOLD, constants.rs:25
    std::vector<uint64_t> idx(n);
    for (uint64_t i = 0; i < n; ++i) idx[i] = i;
    shuffle(rng, idx);
    for (int c = 0; c < k; ++c)
      std::memcpy(&cents[(size_t)c * dim], row(idx[c]), sizeof(float) * dim);
  } else {  // k-means++ (kmeans.rs:101-137)
    uint64_t first = rng.index(n);
    std::memcpy(&cents[0], row(first), sizeof(float) * dim);
    std::vector<float> dist(n);
    for (int c = 1; c < k; ++c) {
      parallel_for(n, nthreads, [&](uint64_t i) {
        float m = 3.40282347e38f;  // fold(f32::MAX, f32::min)
        for (int j = 0; j < c; ++j)
          m = std::fmin(m, l2sq_avx2(row(i), &cents[(size_t)j * dim], (size_t)dim));
        dist[i] = m;
      });
      float total = -0.0f;  // distances.iter().sum()
      for (uint64_t i = 0; i < n; ++i) total += dist[i];
      uint64_t sel;
      if (total == 0.0f) {
        sel = rng.index(n);
      } else {
        float r = rng.unit() * total;
        sel = n - 1;
        for (uint64_t i = 0; i < n; ++i) {
          r -= dist[i];
          if (r <= 0.0f) {
            sel = i;
            break;
          }
        }
      }
      std::memcpy(&cents[(size_t)c * dim], row(sel), sizeof(float) * dim);
    }
  }
  std::vector<int> assign(n);
  std::vector<float> next((size_t)k * dim);
  for (int it = 0; it < max_iters; ++it) {
    parallel_for(n, nthreads, [&](uint64_t i) { assign[i] = nearest(row(i), cents.data(), k, dim); });
    // mean in f32, members visited in index order, then divided by the count
    parallel_for((uint64_t)k, nthreads, [&](uint64_t c) {
      float* mean = &next[c * dim];
      for (int j = 0; j < dim; ++j) mean[j] = 0.0f;
      uint64_t count = 0;
      for (uint64_t i = 0; i < n; ++i) {
        if (assign[i] != (int)c) continue;
        const float* r = row(i);
        for (int j = 0; j < dim; ++j) mean[j] += r[j];
        ++count;
      }
      if (count == 0) {
        std::memcpy(mean, &cents[c * dim], sizeof(float) * dim);
        return;
      }
      float cnt = (float)count;
      for (int j = 0; j < dim; ++j) mean[j] /= cnt;
    });
    // measure_change, kmeans.rs:320-329
    float total = -0.0f;
    for (int c = 0; c < k; ++c)
      total += l2sq_avx2(&cents[(size_t)c * dim], &next[(size_t)c * dim], (size_t)dim);
    float change = total / (float)k;
    cents.swap(next);
    if (change < 0.001f) break;  // CONVERGENCE_THRESHOLD, constants.rs:29
  }
  std::memcpy(out, cents.data(), sizeof(float) * cents.size());
  return 0;
}

// Max-heap with the reference's insertion rules.  BinaryHeap leaves the order
// among equal distances unspecified; here items compare by (distance, key)
// where key is the row position, so exact ties resolve to the earlier row —
// one of the outcomes the reference can produce, and the one the HIP kernels
// produce.
struct HeapItem {
  uint64_t id;
  float d;
  uint64_t key;
};
inline bool item_lt(float d1, uint64_t k1, float d2, uint64_t k2) {
  return d1 < d2 || (d1 == d2 && k1 < k2);
}
struct HeapLess {
  bool operator()(const HeapItem& a, const HeapItem& b) const { return item_lt(a.d, a.key, b.d, b.key); }
};
using MaxHeap = std::priority_queue<HeapItem, std::vector<HeapItem>, HeapLess>;

// heap.into_iter() then a stable ascending sort_by (ivf_pq.rs:673-674)
int heap_to_sorted(MaxHeap& heap, int k, uint64_t* ids, float* dists) {
  std::vector<HeapItem> v;
  v.reserve(heap.size());
  while (!heap.empty()) {
    v.push_back(heap.top());
    heap.pop();
  }
  std::reverse(v.begin(), v.end());
  std::stable_sort(v.begin(), v.end(), [](const HeapItem& a, const HeapItem& b) { return a.d < b.d; });
  int cnt = std::min<int>((int)v.size(), k);
  for (int i = 0; i < cnt; ++i) {
    ids[i] = v[i].id;
    dists[i] = v[i].d;
  }
  return cnt;
}

}  // namespace

// ===========================================================================
// C API
// ===========================================================================
extern "C" {

float fdbo_l2sq(const float* a, const float* b, size_t n) { return l2sq_avx2(a, b, n); }
float fdbo_l2(const float* a, const float* b, size_t n) { return std::sqrt(l2sq_avx2(a, b, n)); }
float fdbo_dot(const float* a, const float* b, size_t n) { return dot_avx2(a, b, n); }
float fdbo_cosine(const float* a, const float* b, size_t n) { return cosine_avx2(a, b, n); }
float fdbo_l1(const float* a, const float* b, size_t n) { return l1_avx2(a, b, n); }

float fdbo_metric(int metric, const float* a, const float* b, size_t n) {
  switch (metric) {
    case FDBO_EUCLIDEAN: return std::sqrt(l2sq_avx2(a, b, n));
    case FDBO_EUCLIDEAN_SQ: return l2sq_avx2(a, b, n);
    case FDBO_COSINE: return cosine_avx2(a, b, n);
    case FDBO_DOT: return -dot_avx2(a, b, n);  // distance/mod.rs:45
    case FDBO_MANHATTAN: return l1_avx2(a, b, n);
  }
  return NAN;
}

// scalar.rs:8-97 — sequential iterator sums
float fdbo_scalar_l2sq(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; ++i) {
    float d = a[i] - b[i];
    s += d * d;
  }
  return s;
}
float fdbo_scalar_dot(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; ++i) s += a[i] * b[i];
  return s;
}
float fdbo_scalar_cosine(const float* a, const float* b, size_t n) {
  float dot = 0.0f, na = 0.0f, nb = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    dot += a[i] * b[i];
    na += a[i] * a[i];
    nb += b[i] * b[i];
  }
  float denom = std::sqrt(na * nb);
  float sim = denom == 0.0f ? 0.0f : dot / denom;
  return 1.0f - sim;  // scalar.rs:86-88: a zero vector gives 1 here, 0 on AVX2
}
float fdbo_scalar_l1(const float* a, const float* b, size_t n) {
  float s = -0.0f;
  for (size_t i = 0; i < n; ++i) s += std::fabs(a[i] - b[i]);
  return s;
}

void fdbo_pq_lut(const float* cb, int M, int dsub, const float* r, float* lut) {
  pq_lut(cb, M, dsub, r, lut);
}
float fdbo_adc_lanes8(const float* lut, const uint8_t* code, int M) { return adc_lanes8(lut, code, M); }
float fdbo_adc_groups4(const float* lut, const uint8_t* code, int M) { return adc_groups4(lut, code, M); }
float fdbo_adc_seq(const float* lut, const uint8_t* code, int M) { return adc_seq(lut, code, M); }
void fdbo_adc_batch4(const float* const* luts, const uint8_t* code, int M, float* out4) {
  adc_batch(luts, 4, code, M, out4);
}
void fdbo_pq_encode(const float* cb, int M, int dsub, const float* x, uint8_t* code) {
  pq_encode(cb, M, dsub, x, code);
}

uint64_t fdbo_splitmix64_at(uint64_t seed, uint64_t i) { return splitmix64_at(seed, i); }
void fdbo_shuffle_indices(uint64_t seed, uint64_t* idx, uint64_t n) {
  Stream rng(seed);
  std::vector<uint64_t> v(idx, idx + n);
  shuffle(rng, v);
  std::memcpy(idx, v.data(), sizeof(uint64_t) * n);
}

int fdbo_kmeans_fit(const float* data, uint64_t n, int dim, int k, int max_iters, uint64_t seed,
                    float* centroids_out) {
  return kmeans_fit(data, n, dim, k, max_iters, seed, centroids_out, 0);
}

// ---------------------------------------------------------------------------
// IVF-PQ
// ---------------------------------------------------------------------------
struct fdbo_ivfpq {
  int nlist, dim, M, dsub;
  std::vector<float> centroids;  // [nlist][dim]
  std::vector<float> codebooks;  // [M][256][dsub]
  std::vector<uint64_t> offsets; // [nlist+1]
  std::vector<uint64_t> ids;     // [N], list order
  std::vector<uint8_t> codes;    // [N][M], list order
  std::atomic<uint64_t> nprobe{1};
  // original_vectors: Option<RwLock<HashMap<u64, Vector>>> (ivf_pq.rs:356)
  bool reranking = false;
  std::unordered_map<uint64_t, std::vector<float>> originals;
  uint64_t rerank_factor = 1;
  // PartitionData::tombstones (ivf_pq.rs:190): ids per list; sized on first use
  std::vector<std::unordered_set<uint64_t>> tomb;
};

namespace {
inline bool tombstoned(const fdbo_ivfpq* h, int list, uint64_t id) {
  return !h->tomb.empty() && h->tomb[list].count(id) != 0;
}
}  // namespace

fdbo_ivfpq* fdbo_ivfpq_create(const float* centroids, int nlist, int dim, const float* codebooks,
                              int M, const uint64_t* list_offsets, const uint64_t* ids,
                              const uint8_t* codes) {
  if (nlist <= 0 || dim <= 0 || M <= 0 || dim % M != 0) return nullptr;
  auto* h = new fdbo_ivfpq();
  h->nlist = nlist;
  h->dim = dim;
  h->M = M;
  h->dsub = dim / M;
  h->centroids.assign(centroids, centroids + (size_t)nlist * dim);
  h->codebooks.assign(codebooks, codebooks + (size_t)M * 256 * h->dsub);
  h->offsets.assign(list_offsets, list_offsets + nlist + 1);
  uint64_t n = h->offsets[nlist];
  h->ids.assign(ids, ids + n);
  h->codes.assign(codes, codes + n * (uint64_t)M);
  return h;
}

// IVFPQIndex::build, ivf_pq.rs:374-506, with seeded sampling streams:
//   splitmix64_at(seed, 0): training-sample shuffle   (:383-396)
//   splitmix64_at(seed, 1): coarse k-means init        (:398-400)
//   splitmix64_at(seed, 2): PQ residual-sample shuffle (:422-446)
//   splitmix64_at(seed, 16 + m): PQ k-means init, subspace m (pq.rs:71-87)
fdbo_ivfpq* fdbo_ivfpq_build(const float* vectors, uint64_t n, int dim, int nlist, int M,
                             uint64_t seed, int nthreads) {
  if (n == 0 || nlist <= 0 || dim <= 0 || M <= 0 || dim % M != 0) return nullptr;
  const int dsub = dim / M;
  auto row = [&](uint64_t i) { return vectors + i * (uint64_t)dim; };
  // 1. coarse training sample
  uint64_t ts = std::min<uint64_t>(n, 30000);
  std::vector<float> sample;
  if (n <= ts) {
    sample.assign(vectors, vectors + n * dim);
  } else {
    Stream rng(splitmix64_at(seed, 0));
    std::vector<uint64_t> idx(n);
    for (uint64_t i = 0; i < n; ++i) idx[i] = i;
    shuffle(rng, idx);
    sample.resize(ts * dim);
    for (uint64_t i = 0; i < ts; ++i) std::memcpy(&sample[i * dim], row(idx[i]), sizeof(float) * dim);
  }
  std::vector<float> cents((size_t)nlist * dim);
  if (kmeans_fit(sample.data(), ts, dim, nlist, 25, splitmix64_at(seed, 1), cents.data(), nthreads))
    return nullptr;
  // 2. assignment
  std::vector<int> assign(n);
  parallel_for(n, nthreads, [&](uint64_t i) { assign[i] = nearest(row(i), cents.data(), nlist, dim); });
  // 3. PQ on residuals of a shuffled sample
  uint64_t ps = std::min<uint64_t>(n, 100000);
  if (ps < 256) return nullptr;
  std::vector<float> resid(ps * dim);
  {
    Stream rng(splitmix64_at(seed, 2));
    std::vector<uint64_t> idx(n);
    for (uint64_t i = 0; i < n; ++i) idx[i] = i;
    shuffle(rng, idx);
    for (uint64_t s = 0; s < ps; ++s) {
      const float* v = row(idx[s]);
      const float* c = &cents[(size_t)assign[idx[s]] * dim];
      for (int j = 0; j < dim; ++j) resid[s * dim + j] = v[j] - c[j];
    }
  }
  std::vector<float> cb((size_t)M * 256 * dsub);
  std::vector<float> sub(ps * dsub);
  for (int m = 0; m < M; ++m) {
    for (uint64_t s = 0; s < ps; ++s)
      std::memcpy(&sub[s * dsub], &resid[s * dim + (size_t)m * dsub], sizeof(float) * dsub);
    if (kmeans_fit(sub.data(), ps, dsub, 256, 25, splitmix64_at(seed, 16 + (uint64_t)m),
                   &cb[(size_t)m * 256 * dsub], nthreads))
      return nullptr;
  }
  // 4. lists in vector order, codes of the residuals
  std::vector<uint64_t> offsets(nlist + 1, 0);
  for (uint64_t i = 0; i < n; ++i) offsets[assign[i] + 1]++;
  for (int l = 0; l < nlist; ++l) offsets[l + 1] += offsets[l];
  std::vector<uint64_t> fill(offsets.begin(), offsets.end() - 1);
  std::vector<uint64_t> order(n);
  for (uint64_t i = 0; i < n; ++i) order[fill[assign[i]]++] = i;
  std::vector<uint64_t> ids(n);
  std::vector<uint8_t> codes(n * M);
  parallel_for(n, nthreads, [&](uint64_t p) {
    uint64_t i = order[p];
    ids[p] = i;
    const float* c = &cents[(size_t)assign[i] * dim];
    std::vector<float> r(dim);
    for (int j = 0; j < dim; ++j) r[j] = row(i)[j] - c[j];
    pq_encode(cb.data(), M, dsub, r.data(), &codes[p * M]);
  });
  return fdbo_ivfpq_create(cents.data(), nlist, dim, cb.data(), M, offsets.data(), ids.data(),
                           codes.data());
}

void fdbo_ivfpq_destroy(fdbo_ivfpq* h) { delete h; }

void fdbo_ivfpq_shape(const fdbo_ivfpq* h, int* nlist, int* dim, int* M, uint64_t* n) {
  *nlist = h->nlist;
  *dim = h->dim;
  *M = h->M;
  *n = h->offsets.back();
}

void fdbo_ivfpq_export(const fdbo_ivfpq* h, float* centroids, float* codebooks,
                       uint64_t* list_offsets, uint64_t* ids, uint8_t* codes) {
  if (centroids) std::memcpy(centroids, h->centroids.data(), h->centroids.size() * 4);
  if (codebooks) std::memcpy(codebooks, h->codebooks.data(), h->codebooks.size() * 4);
  if (list_offsets) std::memcpy(list_offsets, h->offsets.data(), h->offsets.size() * 8);
  if (ids) std::memcpy(ids, h->ids.data(), h->ids.size() * 8);
  if (codes) std::memcpy(codes, h->codes.data(), h->codes.size());
}

void fdbo_ivfpq_set_nprobe(fdbo_ivfpq* h, uint64_t nprobe) {
  h->nprobe.store(std::min<uint64_t>(nprobe, (uint64_t)h->nlist), std::memory_order_relaxed);
}
uint64_t fdbo_ivfpq_nprobe(const fdbo_ivfpq* h) { return h->nprobe.load(std::memory_order_relaxed); }

void fdbo_ivfpq_enable_reranking(fdbo_ivfpq* h, const float* v, uint64_t factor) {
  // enable_reranking (:513-517): the vectors collected into a map by id (a
  // later vector of an id replaces an earlier one), factor at least 1
  h->originals.clear();
  for (uint64_t p = 0; p < h->offsets.back(); ++p)
    h->originals[h->ids[p]].assign(v + p * h->dim, v + (p + 1) * h->dim);
  h->reranking = true;
  h->rerank_factor = std::max<uint64_t>(factor, 1);
}

// from_serializable (ivf_pq.rs:1918-1925, 1940): original_vectors from
// (id, vector) records, a later record of an id replacing an earlier one;
// the rerank factor as stored
void fdbo_ivfpq_set_originals(fdbo_ivfpq* h, const uint64_t* ids, const float* v, uint64_t n,
                              uint64_t factor) {
  h->originals.clear();
  for (uint64_t i = 0; i < n; ++i) h->originals[ids[i]].assign(v + i * h->dim, v + (i + 1) * h->dim);
  h->reranking = true;
  h->rerank_factor = factor;
}

namespace {
// The `count` smallest centroid distances; exact ties resolve to the lower
// centroid index.  select_nth_unstable_by leaves that order unspecified, so
// this is one of the orders the reference can return.  Returns count.
int select_probes(const fdbo_ivfpq* h, const float* q, uint64_t count, int32_t* lists,
                  float* dists) {
  std::vector<std::pair<float, int>> cd(h->nlist);
  for (int c = 0; c < h->nlist; ++c)
    cd[c] = {l2sq_avx2(q, &h->centroids[(size_t)c * h->dim], (size_t)h->dim), c};
  int cnt = (int)std::min<uint64_t>(count, (uint64_t)h->nlist);
  std::partial_sort(cd.begin(), cd.begin() + cnt, cd.end());
  for (int i = 0; i < cnt; ++i) {
    lists[i] = cd[i].second;
    if (dists) dists[i] = cd[i].first;
  }
  return cnt;
}

// rerank_results, ivf_pq.rs:556-582: exact sqrt(l2sq) on original vectors,
// then a stable ascending sort and truncation.  Originals are addressed by
// list position here; the reference looks them up by id.
int rerank(const fdbo_ivfpq* h, const float* q, std::vector<std::pair<uint64_t, float>>& cand,
           int k, uint64_t* out_ids, float* out_d) {
  std::vector<std::pair<uint64_t, float>> rr;
  for (size_t i = 0; i < cand.size(); ++i) {
    auto it = h->originals.find(cand[i].first);  // filter_map: no vector, no result
    if (it == h->originals.end()) continue;
    rr.push_back({cand[i].first, std::sqrt(l2sq_avx2(q, it->second.data(), (size_t)h->dim))});
  }
  std::stable_sort(rr.begin(), rr.end(), [](auto& a, auto& b) { return a.second < b.second; });
  int cnt = std::min<int>((int)rr.size(), k);
  for (int i = 0; i < cnt; ++i) {
    out_ids[i] = rr[i].first;
    out_d[i] = rr[i].second;
  }
  return cnt;
}

struct PosItem {
  uint64_t pos;
  float d;
};
// ordered by (distance, list position); see HeapItem
struct PosLess {
  bool operator()(const PosItem& a, const PosItem& b) const { return item_lt(a.d, a.pos, b.d, b.pos); }
};
using PosHeap = std::priority_queue<PosItem, std::vector<PosItem>, PosLess>;

// the reference's "dist < threshold || len < fetch_k" with the pair order;
// threshold is (f32::MAX, max) while the heap is not full
struct Threshold {
  float d;
  uint64_t pos;
};
inline Threshold threshold_of(const PosHeap& heap, uint64_t fetch_k) {
  if (heap.size() >= fetch_k && !heap.empty()) return {heap.top().d, heap.top().pos};
  return {3.40282347e38f, ~0ull};
}

// heap contents, stable-sorted ascending, then rerank or truncate
int finish(const fdbo_ivfpq* h, const float* q, PosHeap& heap, int k, uint64_t* out_ids,
           float* out_d) {
  std::vector<PosItem> v;
  while (!heap.empty()) {
    v.push_back(heap.top());
    heap.pop();
  }
  std::reverse(v.begin(), v.end());
  std::stable_sort(v.begin(), v.end(), [](const PosItem& a, const PosItem& b) { return a.d < b.d; });
  if (h->reranking) {
    std::vector<std::pair<uint64_t, float>> cand;
    for (auto& it : v) cand.push_back({h->ids[it.pos], it.d});
    return rerank(h, q, cand, k, out_ids, out_d);
  }
  int cnt = std::min<int>((int)v.size(), k);
  for (int i = 0; i < cnt; ++i) {
    out_ids[i] = h->ids[v[i].pos];
    out_d[i] = v[i].d;
  }
  return cnt;
}
}  // namespace

int fdbo_ivfpq_probes(const fdbo_ivfpq* h, const float* q, uint64_t nprobe, int32_t* out_lists,
                      float* out_dists) {
  return select_probes(h, q, nprobe, out_lists, out_dists);
}

// IVFPQIndex::search, ivf_pq.rs:590-677
int fdbo_ivfpq_search(const fdbo_ivfpq* h, const float* q, int k, uint64_t* out_ids,
                      float* out_dists) {
  const uint64_t fetch_k = !h->reranking ? (uint64_t)k : (uint64_t)k * h->rerank_factor;
  uint64_t nprobe = h->nprobe.load(std::memory_order_relaxed);
  std::vector<int32_t> lists(h->nlist);
  int np = select_probes(h, q, nprobe, lists.data(), nullptr);
  PosHeap heap;
  std::vector<float> resid(h->dim), lut((size_t)h->M * 256);
  for (int pi = 0; pi < np; ++pi) {
    int p = lists[pi];
    const float* c = &h->centroids[(size_t)p * h->dim];
    for (int j = 0; j < h->dim; ++j) resid[j] = q[j] - c[j];
    pq_lut(h->codebooks.data(), h->M, h->dsub, resid.data(), lut.data());
    // threshold read once per list (:638-642)
    const Threshold th = threshold_of(heap, fetch_k);
    for (uint64_t j = h->offsets[p]; j < h->offsets[p + 1]; ++j) {
      if (tombstoned(h, p, h->ids[j])) continue;  // :657-659
      float dist = adc_groups4(lut.data(), &h->codes[j * h->M], h->M);
      if (item_lt(dist, j, th.d, th.pos) || heap.size() < fetch_k) {
        heap.push({j, dist});
        if (heap.size() > fetch_k) heap.pop();
      }
    }
  }
  return finish(h, q, heap, k, out_ids, out_dists);
}

// IVFPQIndex::batch_search, ivf_pq.rs:850-1047.  Lists are visited in
// ascending id (the reference's HashMap order is random per process).
void fdbo_ivfpq_batch_search(const fdbo_ivfpq* h, const float* queries, uint64_t nq, int k,
                             uint64_t* out_ids, float* out_dists, int32_t* out_counts) {
  if (nq == 0) return;
  const uint64_t fetch_k = !h->reranking ? (uint64_t)k : (uint64_t)k * h->rerank_factor;
  const int dim = h->dim, M = h->M;
  uint64_t nprobe = h->nprobe.load(std::memory_order_relaxed);
  // [..=nth] with nth = min(nprobe, nlist).saturating_sub(1): nprobe 0 probes 1 list (:877-881)
  uint64_t np = std::max<uint64_t>(1, std::min<uint64_t>(nprobe, (uint64_t)h->nlist));
  std::map<int, std::vector<uint64_t>> part_queries;
  std::vector<int32_t> lists(np);
  for (uint64_t qi = 0; qi < nq; ++qi) {
    select_probes(h, queries + qi * dim, np, lists.data(), nullptr);
    for (uint64_t i = 0; i < np; ++i) part_queries[lists[i]].push_back(qi);
  }
  std::vector<PosHeap> heaps(nq);
  std::vector<float> resid(dim);
  for (auto& kv : part_queries) {
    int p = kv.first;
    const std::vector<uint64_t>& qidx = kv.second;
    const float* c = &h->centroids[(size_t)p * dim];
    std::vector<std::vector<float>> tables(qidx.size(), std::vector<float>((size_t)M * 256));
    for (size_t t = 0; t < qidx.size(); ++t) {
      const float* q = queries + qidx[t] * dim;
      for (int j = 0; j < dim; ++j) resid[j] = q[j] - c[j];
      pq_lut(h->codebooks.data(), M, h->dsub, resid.data(), tables[t].data());
    }
    std::vector<const float*> refs(qidx.size());
    for (size_t t = 0; t < qidx.size(); ++t) refs[t] = tables[t].data();
    const bool use_batch = qidx.size() >= 4;
    std::vector<float> dists(qidx.size());
    for (uint64_t j = h->offsets[p]; j < h->offsets[p + 1]; ++j) {
      if (tombstoned(h, p, h->ids[j])) continue;  // :960-963
      const uint8_t* code = &h->codes[j * M];
      if (use_batch) {
        adc_batch(refs.data(), (int)refs.size(), code, M, dists.data());
      } else {
        for (size_t t = 0; t < qidx.size(); ++t) dists[t] = adc_lanes8(refs[t], code, M);
      }
      for (size_t t = 0; t < qidx.size(); ++t) {
        PosHeap& heap = heaps[qidx[t]];
        const Threshold th = threshold_of(heap, fetch_k);
        float dist = dists[t];
        if (item_lt(dist, j, th.d, th.pos) || heap.size() < fetch_k) {
          heap.push({j, dist});
          if (heap.size() > fetch_k) heap.pop();
        }
      }
    }
  }
  for (uint64_t qi = 0; qi < nq; ++qi)
    out_counts[qi] = finish(h, queries + qi * dim, heaps[qi], k, out_ids + qi * (uint64_t)k,
                            out_dists + qi * (uint64_t)k);
}

// search_filtered, ivf_pq.rs:692-831: the filter as the set of admitted ids.
// Heap of 4 * fetch_k, threshold read once per list, tombstoned and
// unadmitted entries skipped, then rerank or truncation.
int fdbo_ivfpq_search_filtered(const fdbo_ivfpq* h, const float* q, int k, const uint64_t* allowed,
                               uint64_t n_allowed, uint64_t* out_ids, float* out_dists) {
  if (n_allowed == 0) return 0;  // :700-703
  std::unordered_set<uint64_t> allow(allowed, allowed + n_allowed);
  const uint64_t fetch_k = !h->reranking ? (uint64_t)k : (uint64_t)k * h->rerank_factor;
  const uint64_t filter_fetch_k = fetch_k * 4;  // :712
  uint64_t nprobe = h->nprobe.load(std::memory_order_relaxed);
  std::vector<int32_t> lists(h->nlist);
  int np = select_probes(h, q, nprobe, lists.data(), nullptr);
  PosHeap heap;
  std::vector<float> resid(h->dim), lut((size_t)h->M * 256);
  for (int pi = 0; pi < np; ++pi) {
    int p = lists[pi];
    const float* c = &h->centroids[(size_t)p * h->dim];
    for (int j = 0; j < h->dim; ++j) resid[j] = q[j] - c[j];
    pq_lut(h->codebooks.data(), h->M, h->dsub, resid.data(), lut.data());
    const Threshold th = threshold_of(heap, filter_fetch_k);
    for (uint64_t j = h->offsets[p]; j < h->offsets[p + 1]; ++j) {
      if (tombstoned(h, p, h->ids[j]) || !allow.count(h->ids[j])) continue;
      float dist = adc_groups4(lut.data(), &h->codes[j * h->M], h->M);
      if (item_lt(dist, j, th.d, th.pos) || heap.size() < filter_fetch_k) {
        heap.push({j, dist});
        if (heap.size() > filter_fetch_k) heap.pop();
      }
    }
  }
  return finish(h, q, heap, k, out_ids, out_dists);
}

// delete, ivf_pq.rs:1786-1804
int fdbo_ivfpq_delete(fdbo_ivfpq* h, uint64_t id) {
  if (h->tomb.empty()) h->tomb.resize(h->nlist);
  for (int l = 0; l < h->nlist; ++l) {
    if (h->tomb[l].count(id)) continue;
    for (uint64_t j = h->offsets[l]; j < h->offsets[l + 1]; ++j)
      if (h->ids[j] == id) {
        h->tomb[l].insert(id);
        if (h->reranking) h->originals.erase(id);  // :1793-1797
        return 1;
      }
  }
  return 0;
}

uint64_t fdbo_ivfpq_num_tombstones(const fdbo_ivfpq* h) {
  uint64_t n = 0;
  for (auto& t : h->tomb) n += t.size();
  return n;
}

// insert_batch, ivf_pq.rs:1731-1776, one vector at a time in input order
void fdbo_ivfpq_insert(fdbo_ivfpq* h, const float* vectors, const uint64_t* ids, uint64_t n) {
  if (h->tomb.empty()) h->tomb.resize(h->nlist);
  const int dim = h->dim, M = h->M;
  std::vector<float> resid(dim);
  std::vector<uint8_t> code(M);
  for (uint64_t i = 0; i < n; ++i) {
    const float* v = vectors + i * (uint64_t)dim;
    const int l = nearest(v, h->centroids.data(), h->nlist, dim);
    const float* c = &h->centroids[(size_t)l * dim];
    for (int j = 0; j < dim; ++j) resid[j] = v[j] - c[j];
    pq_encode(h->codebooks.data(), M, h->dsub, resid.data(), code.data());
    const uint64_t at = h->offsets[l + 1];
    h->ids.insert(h->ids.begin() + at, ids[i]);
    h->codes.insert(h->codes.begin() + at * M, code.begin(), code.end());
    if (h->reranking) h->originals[ids[i]].assign(v, v + dim);  // :1769-1773
    for (int t = l + 1; t <= h->nlist; ++t) h->offsets[t]++;
    h->tomb[l].erase(ids[i]);
  }
}

// compact, ivf_pq.rs:1828-1851
void fdbo_ivfpq_compact(fdbo_ivfpq* h) {
  if (h->tomb.empty()) return;
  const int M = h->M;
  std::vector<uint64_t> offs(h->nlist + 1, 0), ids;
  std::vector<uint8_t> codes;
  for (int l = 0; l < h->nlist; ++l) {
    for (uint64_t j = h->offsets[l]; j < h->offsets[l + 1]; ++j) {
      if (h->tomb[l].count(h->ids[j])) continue;
      ids.push_back(h->ids[j]);
      codes.insert(codes.end(), &h->codes[j * M], &h->codes[j * M] + M);
    }
    offs[l + 1] = ids.size();
    h->tomb[l].clear();
  }
  h->offsets.swap(offs);
  h->ids.swap(ids);
  h->codes.swap(codes);
}

// batch_search_parallel, ivf_pq.rs:1060-1084
void fdbo_ivfpq_batch_search_parallel(const fdbo_ivfpq* h, const float* queries, uint64_t nq,
                                      int k, int nthreads, uint64_t* out_ids, float* out_dists,
                                      int32_t* out_counts) {
  if (nq == 0) return;
  uint64_t nprobe = h->nprobe.load(std::memory_order_relaxed);
  uint64_t table_bytes = (uint64_t)h->M * 256 * 4;
  uint64_t chunk = (256 * 1024) / (std::max<uint64_t>(nprobe, 1) * table_bytes);
  chunk = std::min<uint64_t>(std::max<uint64_t>(chunk, 4), 64);
  uint64_t nchunks = (nq + chunk - 1) / chunk;
  parallel_for(nchunks, nthreads, [&](uint64_t c) {
    uint64_t q0 = c * chunk, cnt = std::min(chunk, nq - q0);
    fdbo_ivfpq_batch_search(h, queries + q0 * h->dim, cnt, k, out_ids + q0 * (uint64_t)k,
                            out_dists + q0 * (uint64_t)k, out_counts + q0);
  });
}

// ---------------------------------------------------------------------------
// Brute force, brute_force.rs:105-225
// ---------------------------------------------------------------------------
namespace {
// scan_range, :105-148: push while len < k, else replace the max only when
// smaller (in (distance, row) order: a later row never displaces an equal
// earlier one, as with the reference's strict `<` in a sequential scan).
void bf_scan(const float* data, const uint64_t* ids, int dim, int metric, const float* q,
             uint64_t start, uint64_t end, MaxHeap& heap, int k) {
  for (uint64_t i = start; i < end; ++i) {
    float d = fdbo_metric(metric, q, data + i * (uint64_t)dim, (size_t)dim);
    if ((int)heap.size() < k) {
      heap.push({ids[i], d, i});
    } else if (!heap.empty() && item_lt(d, i, heap.top().d, heap.top().key)) {
      heap.pop();
      heap.push({ids[i], d, i});
    }
  }
}
}  // namespace

int fdbo_bf_search(const float* data, const uint64_t* ids, uint64_t n, int dim, int metric,
                   const float* q, int k, uint64_t* out_ids, float* out_dists) {
  MaxHeap heap;
  bf_scan(data, ids, dim, metric, q, 0, n, heap, k);
  return heap_to_sorted(heap, k, out_ids, out_dists);
}

// search_parallel, :180-214: 1000-row chunks (BRUTE_FORCE_CHUNK_SIZE,
// constants.rs:58), folded with the same rule.
int fdbo_bf_search_parallel(const float* data, const uint64_t* ids, uint64_t n, int dim,
                            int metric, const float* q, int k, uint64_t* out_ids,
                            float* out_dists) {
  MaxHeap acc;
  const uint64_t chunk = 1000;
  for (uint64_t s = 0; s < n; s += chunk) {
    MaxHeap local;
    bf_scan(data, ids, dim, metric, q, s, std::min(n, s + chunk), local, k);
    while (!local.empty()) {
      HeapItem it = local.top();
      local.pop();
      if ((int)acc.size() < k) {
        acc.push(it);
      } else if (!acc.empty() && item_lt(it.d, it.key, acc.top().d, acc.top().key)) {
        acc.pop();
        acc.push(it);
      }
    }
  }
  return heap_to_sorted(acc, k, out_ids, out_dists);
}

// batch_search, :220-225: queries in parallel, each a search_parallel
void fdbo_bf_batch_search(const float* data, const uint64_t* ids, uint64_t n, int dim, int metric,
                          const float* queries, uint64_t nq, int k, int nthreads,
                          uint64_t* out_ids, float* out_dists, int32_t* out_counts) {
  parallel_for(nq, nthreads, [&](uint64_t qi) {
    out_counts[qi] = fdbo_bf_search_parallel(data, ids, n, dim, metric, queries + qi * dim, k,
                                             out_ids + qi * (uint64_t)k,
                                             out_dists + qi * (uint64_t)k);
  });
}

// ---------------------------------------------------------------------------
// IVF-flat, ivf.rs:162-216 (coarse is a stable full sort of l2sq; the scan
// uses the index metric and the brute-force heap rule)
// ---------------------------------------------------------------------------
int fdbo_ivf_probes(const float* centroids, int nlist, int dim, const float* q, uint64_t nprobe,
                    int32_t* out_lists) {
  std::vector<std::pair<float, int>> cd(nlist);
  for (int c = 0; c < nlist; ++c)
    cd[c] = {l2sq_avx2(q, centroids + (size_t)c * dim, (size_t)dim), c};
  std::stable_sort(cd.begin(), cd.end(),
                   [](auto& a, auto& b) { return a.first < b.first; });
  int cnt = (int)std::min<uint64_t>(nprobe, (uint64_t)nlist);
  for (int i = 0; i < cnt; ++i) out_lists[i] = cd[i].second;
  return cnt;
}

int fdbo_ivf_search(const float* centroids, int nlist, int dim, const uint64_t* offs,
                    const uint64_t* ids, const float* rows, int metric, uint64_t nprobe,
                    const float* q, int k, uint64_t* out_ids, float* out_dists) {
  std::vector<int32_t> lists(nlist);
  int np = fdbo_ivf_probes(centroids, nlist, dim, q, nprobe, lists.data());
  MaxHeap heap;
  for (int i = 0; i < np; ++i) {
    int p = lists[i];
    bf_scan(rows, ids, dim, metric, q, offs[p], offs[p + 1], heap, k);
  }
  return heap_to_sorted(heap, k, out_ids, out_dists);
}

// batch_search, ivf.rs:292-297: queries in parallel
void fdbo_ivf_batch_search(const float* centroids, int nlist, int dim, const uint64_t* offs,
                           const uint64_t* ids, const float* rows, int metric, uint64_t nprobe,
                           const float* queries, uint64_t nq, int k, int nthreads,
                           uint64_t* out_ids, float* out_dists, int32_t* out_counts) {
  parallel_for(nq, nthreads, [&](uint64_t qi) {
    out_counts[qi] = fdbo_ivf_search(centroids, nlist, dim, offs, ids, rows, metric, nprobe,
                                     queries + qi * dim, k, out_ids + qi * (uint64_t)k,
                                     out_dists + qi * (uint64_t)k);
  });
}

// IVFIndex::build (ivf.rs:91-119): KMeans::new(n_clusters,
// DEFAULT_MAX_ITERATIONS = 100) fitted on every vector, seeded from
// splitmix64_at(seed, 1); each vector to its first-minimum squared-L2
// centroid (min_by, ivf.rs:101-108), lists keeping input order.
int fdbo_ivf_build(const float* vectors, uint64_t n, int dim, int nlist, uint64_t seed,
                   int nthreads, float* centroids_out, uint64_t* offsets_out,
                   uint64_t* order_out) {
  if (n == 0 || nlist <= 0 || dim <= 0) return -1;
  if (kmeans_fit(vectors, n, dim, nlist, 100, splitmix64_at(seed, 1), centroids_out, nthreads))
    return -1;
  std::vector<int> assign(n);
  parallel_for(n, nthreads, [&](uint64_t i) {
    assign[i] = nearest(vectors + i * (uint64_t)dim, centroids_out, nlist, dim);
  });
  std::fill(offsets_out, offsets_out + nlist + 1, 0);
  for (uint64_t i = 0; i < n; ++i) offsets_out[assign[i] + 1]++;
  for (int l = 0; l < nlist; ++l) offsets_out[l + 1] += offsets_out[l];
  std::vector<uint64_t> fill(offsets_out, offsets_out + nlist);
  for (uint64_t i = 0; i < n; ++i) order_out[fill[assign[i]]++] = i;
  return 0;
}

}  // extern "C"
