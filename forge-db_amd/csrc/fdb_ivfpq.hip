// IVF-PQ index: device layout, search orchestration, GPU build.
#include "fdb_ivfpq.hpp"

#include <algorithm>
#include <cstring>
#include <unordered_map>

#include "fdb_device.hpp"
#include "fdb_kernels.hpp"

namespace fdb {

namespace {

__global__ void fill_empty_kernel(uint64_t n, uint32_t k, uint64_t* ids, float* dists,
                                  uint32_t* counts) {
  const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n * k) {
    ids[e] = ~0ull;
    dists[e] = f_inf();
  }
  if (e < n) counts[e] = 0;
}

__global__ void iota_probes_kernel(uint64_t nq, uint32_t np, int32_t* probes) {
  const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < nq * np) probes[e] = (int32_t)(e % np);
}

__global__ void clear_int_kernel(int* p) { *p = 0; }

// Every list is probed (nprobe >= nlist): no selection runs, but a NaN query
// still has to be reported as the reference's comparison would panic on it.
__global__ void nan_check_kernel(const float* __restrict__ q, uint64_t n, int* err) {
  const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < n && q[e] != q[e]) atomicOr(err, 1);
}

// rerank_results, ivf_pq.rs:556-582: candidates arrive sorted by ADC
// distance; each gets sqrt of the exact reference-order squared L2 to its
// original vector, and a stable ascending sort of those (ties keep the ADC
// order: the tie key is the candidate's rank) is truncated to k.  Entries
// whose bit in orig_bits is clear (null: every entry has one) have no
// original and are left out.  One wave per query.
template <int R>
__global__ __launch_bounds__(64) void rerank_kernel(const float* __restrict__ queries, int dim,
                                                    const float* __restrict__ originals,
                                                    const uint32_t* __restrict__ orig_bits,
                                                    const uint64_t* __restrict__ ids,
                                                    const uint32_t* __restrict__ cand_pos,
                                                    const uint32_t* __restrict__ cand_cnt,
                                                    uint32_t fetch_k, uint32_t k,
                                                    uint64_t* __restrict__ out_ids,
                                                    float* __restrict__ out_dists,
                                                    uint32_t* __restrict__ out_counts) {
  const uint64_t q = blockIdx.x;
  const int lane = threadIdx.x;
  const float* __restrict__ qv = queries + q * dim;
  const uint32_t cnt = cand_cnt[q];
  WaveTopK<R> tk;
  tk.init((int)k);
  for (uint32_t base = 0; base < cnt; base += 64) {
    const uint32_t c = base + lane;
    float d = f_inf();
    uint32_t rank = kNoPos;
    if (c < cnt) {
      const uint32_t pos = cand_pos[q * fetch_k + c];
      // an entry without an original vector is dropped (filter_map)
      if (!orig_bits || ((orig_bits[pos >> 5] >> (pos & 31)) & 1u)) {
        d = __builtin_sqrtf(l2sq_ref_rt(qv, originals + (uint64_t)pos * dim, dim));
        rank = c;
      }
    }
    tk.offer(d, rank);
  }
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t s = r * 64 + lane;
    const bool valid = s < k && tk.p[r] != kNoPos;
    count += (uint32_t)__popcll(__ballot(valid));
    if (s < k) {
      out_ids[q * k + s] = valid ? ids[cand_pos[q * fetch_k + tk.p[r]]] : ~0ull;
      out_dists[q * k + s] = valid ? tk.d[r] : f_inf();
    }
  }
  if (lane == 0) out_counts[q] = count;
}

// Device scratch of fdb_ivfpq_batch_search_device_noalloc: the probe lists,
// one copy per device, held until the process ends.  Host code uses the
// address hipGetSymbolAddress returns for the current device
// (noalloc_scratch), never the array's name.
constexpr uint64_t kNoAllocProbes = 1ull << 21;  // int32 entries (8 MiB)
__device__ __align__(256) int32_t scratch[kNoAllocProbes];

int regs_for(uint32_t k) {
  int r = (int)((k + 63) / 64), p = 1;
  while (p < r) p <<= 1;
  return p;
}

hipError_t launch_rerank(const float* queries, uint64_t nq, int dim, const float* originals,
                         const uint32_t* orig_bits, const uint64_t* ids, const uint32_t* cand_pos,
                         const uint32_t* cand_cnt, uint32_t fetch_k, uint32_t k, uint64_t* out_ids,
                         float* out_dists, uint32_t* out_counts, hipStream_t s) {
#define FDB_RR(R)                                                                             \
  hipLaunchKernelGGL(rerank_kernel<R>, dim3((unsigned)nq), dim3(64), 0, s, queries, dim,      \
                     originals, orig_bits, ids, cand_pos, cand_cnt, fetch_k, k, out_ids,     \
                     out_dists, out_counts);                                                  \
  break;
  switch (regs_for(k)) {
    case 1: FDB_RR(1)
    case 2: FDB_RR(2)
    case 4: FDB_RR(4)
    case 8: FDB_RR(8)
    case 16: FDB_RR(16)
    default: return hipErrorInvalidValue;
  }
#undef FDB_RR
  return hipGetLastError();
}

unsigned blocks_for(uint64_t n, unsigned t) { return (unsigned)((n + t - 1) / t); }

// The first k of fetch_k sorted candidates per query (the reference's
// truncate(k) after sorting its candidate heap).
__global__ void truncate_kernel(const uint64_t* __restrict__ cid, const float* __restrict__ cd,
                                const uint32_t* __restrict__ ccnt, uint64_t nq, uint32_t fetch_k,
                                uint32_t k, uint64_t* __restrict__ ids, float* __restrict__ d,
                                uint32_t* __restrict__ cnt) {
  const uint64_t e = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= nq * k) return;
  const uint64_t q = e / k, s = e - q * k;
  ids[e] = cid[q * fetch_k + s];
  d[e] = cd[q * fetch_k + s];
  if (s == 0) cnt[q] = ccnt[q] < k ? ccnt[q] : k;
}

hipError_t launch_truncate(const uint64_t* cid, const float* cd, const uint32_t* ccnt, uint64_t nq,
                           uint32_t fetch_k, uint32_t k, uint64_t* ids, float* d, uint32_t* cnt,
                           hipStream_t s) {
  if (nq == 0 || k == 0) return hipSuccess;
  hipLaunchKernelGGL(truncate_kernel, dim3(blocks_for(nq * k, 256)), dim3(256), 0, s, cid, cd, ccnt, nq,
                     fetch_k, k, ids, d, cnt);
  return hipGetLastError();
}

}  // namespace

// The current device's copy of the no-allocation scratch: its address is
// looked up once per device (with that device current) and kept.
int32_t* noalloc_scratch(uint64_t& cap) {
  static std::mutex mu;
  static int32_t* addr[64] = {};
  int dev = 0;
  FDB_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) throw Error(FDB_ERR_UNSUPPORTED, "device ordinal above 63");
  std::lock_guard<std::mutex> g(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    FDB_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    addr[dev] = static_cast<int32_t*>(p);
  }
  cap = kNoAllocProbes;
  return addr[dev];
}

// Members of each cluster in ascending point order (a stable counting sort).
void group_members(const std::vector<int32_t>& assign, int k, std::vector<uint32_t>& off,
                   std::vector<uint32_t>& members) {
  for (int32_t a : assign)
    if (a < 0 || a >= k) throw Error(FDB_ERR_NAN, "assignment failed (NaN distance)");
  off.assign(k + 1, 0);
  for (int32_t a : assign) off[a + 1]++;
  for (int c = 0; c < k; ++c) off[c + 1] += off[c];
  std::vector<uint32_t> fill(off.begin(), off.end() - 1);
  members.resize(assign.size());
  for (size_t i = 0; i < assign.size(); ++i) members[fill[assign[i]]++] = (uint32_t)i;
}

// KMeans::fit_raw (kmeans.rs:87-193) with a seeded stream: random-sample
// initialisation above KMEANSPP_THRESHOLD = 64 (constants.rs:25), k-means++
// otherwise; Lloyd steps on the GPU (assignment with the first-minimum rule,
// f32 means summed in point order); stop when the mean squared centroid
// shift (measure_change, kmeans.rs:320-329) is below 0.001
// (CONVERGENCE_THRESHOLD, constants.rs:29).
std::vector<float> kmeans_gpu(const float* h_points, uint64_t n, int dim, int k, int max_iters,
                              uint64_t seed, hipStream_t s) {
  if (n < (uint64_t)k || k <= 0)
    throw Error(FDB_ERR_INVALID_ARGUMENT, "k-means needs at least k training vectors");
  if (n > 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "k-means sample above 2^32 rows");
  Stream rng(seed);
  std::vector<float> cents((size_t)k * dim);
  auto row = [&](uint64_t i) { return h_points + i * (uint64_t)dim; };
  if (k > 64) {
    std::vector<uint64_t> idx(n);
    for (uint64_t i = 0; i < n; ++i) idx[i] = i;
    shuffle(rng, idx);
    for (int c = 0; c < k; ++c) std::memcpy(&cents[(size_t)c * dim], row(idx[c]), 4 * dim);
  } else {
    const uint64_t first = rng.index(n);
    std::memcpy(&cents[0], row(first), 4 * dim);
    std::vector<float> dist(n, 3.40282347e38f);
    for (int c = 1; c < k; ++c) {
      // running min over the centroids chosen so far equals the reference's
      // fold(f32::MAX, f32::min) over all of them
      const float* last = &cents[(size_t)(c - 1) * dim];
      for (uint64_t i = 0; i < n; ++i) dist[i] = std::fmin(dist[i], host_l2sq_ref(row(i), last, dim));
      float total = -0.0f;
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
      std::memcpy(&cents[(size_t)c * dim], row(sel), 4 * dim);
    }
  }
  DevBuf<float> d_pts, d_c, d_cT, d_next;
  DevBuf<int32_t> d_assign;
  DevBuf<uint32_t> d_mem, d_off;
  d_pts.upload(h_points, n * dim, s);
  d_c.reserve((size_t)k * dim);
  d_cT.reserve((size_t)centT_ld(k) * dim);
  d_next.reserve((size_t)k * dim);
  d_assign.reserve(n);
  std::vector<int32_t> assign(n);
  std::vector<uint32_t> off, members;
  std::vector<float> next((size_t)k * dim);
  for (int it = 0; it < max_iters; ++it) {
    FDB_HIP(hipMemcpyAsync(d_c.p, cents.data(), 4 * cents.size(), hipMemcpyHostToDevice, s));
    FDB_HIP(launch_transpose_centroids(d_c.p, k, dim, d_cT.p, s));
    FDB_HIP(launch_assign(d_pts.p, n, dim, d_cT.p, k, d_assign.p, s));
    FDB_HIP(hipMemcpyAsync(assign.data(), d_assign.p, 4 * n, hipMemcpyDeviceToHost, s));
    FDB_HIP(hipStreamSynchronize(s));
    group_members(assign, k, off, members);
    d_mem.upload(members.data(), members.size(), s);
    d_off.upload(off.data(), off.size(), s);
    FDB_HIP(launch_kmeans_update(d_pts.p, dim, d_mem.p, d_off.p, k, d_c.p, d_next.p, s));
    FDB_HIP(hipMemcpyAsync(next.data(), d_next.p, 4 * next.size(), hipMemcpyDeviceToHost, s));
    FDB_HIP(hipStreamSynchronize(s));
    float total = -0.0f;
    for (int c = 0; c < k; ++c)
      total += host_l2sq_ref(&cents[(size_t)c * dim], &next[(size_t)c * dim], dim);
    const float change = total / (float)k;
    cents.swap(next);
    if (change < 0.001f) break;
  }
  return cents;
}

IvfPqIndex::IvfPqIndex(IvfPqArtifacts&& art) : host_(std::move(art)) {
  // from_serializable keeps the stored value (ivf_pq.rs:1937); every search
  // clamps it to nlist
  nprobe_.store(host_.nprobe, std::memory_order_relaxed);
  order_.init();
  if (host_.has_originals && host_.orig_ok.size() != host_.ids.size()) host_.orig_ok.assign(host_.ids.size(), 1);
  FDB_HIP(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  for (auto& e : ev_) FDB_HIP(hipEventCreate(&e));
  const uint64_t N = host_.ids.size();
  if (N >= 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "more than 2^32-2 vectors");
  centroids_.upload(host_.centroids.data(), host_.centroids.size(), stream_);
  centT_.reserve((size_t)centT_ld(host_.nlist) * host_.dim);
  FDB_HIP(launch_transpose_centroids(centroids_.p, host_.nlist, host_.dim, centT_.p, stream_));
  coarse_.init(centroids_.p, centT_.p, host_.nlist, host_.dim, stream_);
  codebooks_.upload(host_.codebooks.data(), host_.codebooks.size(), stream_);
  cbnorm_.reserve((size_t)host_.M * 256);
  FDB_HIP(launch_codebook_norms(codebooks_.p, host_.M, host_.dsub, cbnorm_.p, stream_));
  tomb_.assign(host_.nlist, {});
  upload_lists();
  err_.reserve(1);
  hipLaunchKernelGGL(clear_int_kernel, dim3(1), dim3(1), 0, stream_, err_.p);
  FDB_HIP(hipGetLastError());
  FDB_HIP(hipStreamSynchronize(stream_));
}

void IvfPqIndex::upload_lists() {
  std::vector<uint32_t> off32(host_.offsets.begin(), host_.offsets.end());
  off_.upload(off32.data(), off32.size(), stream_);
  codes_.reserve(std::max<size_t>(host_.codes.size(), 16));
  if (!host_.codes.empty())
    FDB_HIP(hipMemcpyAsync(codes_.p, host_.codes.data(), host_.codes.size(), hipMemcpyHostToDevice,
                           stream_));
  ids_.upload(host_.ids.data(), std::max<size_t>(host_.ids.size(), 1), stream_);
  upload_originals();
  live_dirty_ = true;
  pq16_dirty_ = true;
  FDB_HIP(hipStreamSynchronize(stream_));
}

void IvfPqIndex::upload_originals() {
  orig_all_ = true;
  if (!host_.has_originals) return;
  const uint64_t N = host_.ids.size();
  if (!host_.originals.empty()) originals_.upload(host_.originals.data(), host_.originals.size(), stream_);
  std::vector<uint32_t> bits((N + 31) / 32, 0);
  for (uint64_t i = 0; i < N; ++i)
    if (host_.orig_ok[i]) bits[i >> 5] |= 1u << (i & 31);
    else orig_all_ = false;
  if (!orig_all_) orig_bits_.upload(bits.data(), bits.size(), stream_);
  FDB_HIP(hipStreamSynchronize(stream_));
}

void IvfPqIndex::set_original(uint64_t id, const float* v) {
  const uint64_t N = host_.ids.size(), dim = host_.dim;
  for (uint64_t p = 0; p < N; ++p)
    if (host_.ids[p] == id) {
      if (v) std::memcpy(&host_.originals[p * dim], v, 4 * dim);
      host_.orig_ok[p] = v ? 1 : 0;
    }
}

const uint32_t* IvfPqIndex::live_bitmap() {
  if (n_tomb_ == 0) return nullptr;
  if (live_dirty_) {
    const uint64_t N = host_.ids.size();
    std::vector<uint32_t> bits((N + 31) / 32, 0xFFFFFFFFu);
    for (uint32_t l = 0; l < host_.nlist; ++l) {
      if (tomb_[l].empty()) continue;
      for (uint64_t p = host_.offsets[l]; p < host_.offsets[l + 1]; ++p)
        if (tomb_[l].count(host_.ids[p])) bits[p >> 5] &= ~(1u << (p & 31));
    }
    live_.upload(bits.data(), std::max<size_t>(bits.size(), 1), stream_);
    FDB_HIP(hipStreamSynchronize(stream_));
    live_dirty_ = false;
  }
  return live_.p;
}

void IvfPqIndex::last_screen_stats(uint64_t& fallbacks, uint64_t& candidates, hipStream_t s) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, s ? s : stream_);
  fallbacks = candidates = 0;
  if (path_ != 2) return;
  FDB_HIP(hipStreamSynchronize(s ? s : stream_));
  pq16s_.read_stats(fallbacks, candidates, s ? s : stream_);
}

void IvfPqIndex::throw_if_nan() {
  int flag = 0;
  FDB_HIP(hipMemcpy(&flag, err_.p, 4, hipMemcpyDeviceToHost));
  if (flag) {
    hipLaunchKernelGGL(clear_int_kernel, dim3(1), dim3(1), 0, stream_, err_.p);
    FDB_HIP(hipStreamSynchronize(stream_));
    throw Error(FDB_ERR_NAN, "NaN centroid distance (a query contains NaN)");
  }
}

bool IvfPqIndex::remove(uint64_t id) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  for (uint32_t l = 0; l < host_.nlist; ++l) {
    if (tomb_[l].count(id)) continue;
    for (uint64_t p = host_.offsets[l]; p < host_.offsets[l + 1]; ++p)
      if (host_.ids[p] == id) {
        tomb_[l].insert(id);
        ++n_tomb_;
        live_dirty_ = true;
        // the id leaves original_vectors (ivf_pq.rs:1793-1797): every entry
        // holding it is left out of reranking from now on
        if (host_.has_originals) {
          set_original(id, nullptr);
          upload_originals();
        }
        return true;
      }
  }
  return false;
}

void IvfPqIndex::compact() {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  if (n_tomb_ == 0) return;
  const uint32_t M = host_.M, dim = host_.dim;
  std::vector<uint64_t> offs(host_.nlist + 1, 0), ids;
  std::vector<uint8_t> codes, ok;
  std::vector<float> orig;
  ids.reserve(host_.ids.size());
  codes.reserve(host_.codes.size());
  for (uint32_t l = 0; l < host_.nlist; ++l) {
    for (uint64_t p = host_.offsets[l]; p < host_.offsets[l + 1]; ++p) {
      if (tomb_[l].count(host_.ids[p])) continue;
      ids.push_back(host_.ids[p]);
      codes.insert(codes.end(), &host_.codes[p * M], &host_.codes[p * M] + M);
      if (host_.has_originals) {
        orig.insert(orig.end(), &host_.originals[p * dim], &host_.originals[p * dim] + dim);
        ok.push_back(host_.orig_ok[p]);
      }
    }
    offs[l + 1] = ids.size();
    tomb_[l].clear();
  }
  host_.offsets.swap(offs);
  host_.ids.swap(ids);
  host_.codes.swap(codes);
  if (host_.has_originals) {
    host_.originals.swap(orig);
    host_.orig_ok.swap(ok);
  }
  n_tomb_ = 0;
  upload_lists();
}

void IvfPqIndex::insert(const float* vectors, const uint64_t* ids, uint64_t n) {
  if (n == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  const uint32_t M = host_.M, dim = host_.dim;
  for (uint64_t i = 0; i < n * dim; ++i)
    if (std::isnan(vectors[i])) throw Error(FDB_ERR_NAN, "NaN in the vectors to insert");
  if (host_.ids.size() + n >= 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "more than 2^32-2 vectors");
  // nearest list (first minimum) and the residual code, on the GPU
  DevBuf<float> d_vec;
  DevBuf<int32_t> d_assign;
  DevBuf<uint64_t> d_rows;
  DevBuf<uint8_t> d_codes;
  std::vector<uint64_t> rows(n);
  for (uint64_t i = 0; i < n; ++i) rows[i] = i;
  d_vec.upload(vectors, n * dim, stream_);
  d_rows.upload(rows.data(), n, stream_);
  d_assign.reserve(n);
  d_codes.reserve(n * M);
  FDB_HIP(launch_assign(d_vec.p, n, dim, centT_.p, host_.nlist, d_assign.p, stream_));
  FDB_HIP(launch_pq_encode(d_vec.p, d_rows.p, d_assign.p, n, dim, centroids_.p, codebooks_.p, M,
                           host_.dsub, d_codes.p, stream_));
  std::vector<int32_t> assign(n);
  std::vector<uint8_t> newc(n * M);
  FDB_HIP(hipMemcpyAsync(assign.data(), d_assign.p, 4 * n, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipMemcpyAsync(newc.data(), d_codes.p, n * M, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
  // each list: its old entries, then the new ones in input order
  std::vector<uint32_t> off, members;
  group_members(assign, (int)host_.nlist, off, members);
  const uint64_t n_old = host_.ids.size();
  std::vector<uint64_t> offs(host_.nlist + 1, 0), nids;
  std::vector<uint8_t> codes, ok;
  std::vector<float> orig;
  nids.reserve(host_.ids.size() + n);
  codes.reserve(host_.codes.size() + n * M);
  for (uint32_t l = 0; l < host_.nlist; ++l) {
    const uint64_t s = host_.offsets[l], e = host_.offsets[l + 1];
    nids.insert(nids.end(), host_.ids.begin() + s, host_.ids.begin() + e);
    codes.insert(codes.end(), host_.codes.begin() + s * M, host_.codes.begin() + e * M);
    if (host_.has_originals) {
      orig.insert(orig.end(), host_.originals.begin() + s * dim, host_.originals.begin() + e * dim);
      ok.insert(ok.end(), host_.orig_ok.begin() + s, host_.orig_ok.begin() + e);
    }
    for (uint32_t t = off[l]; t < off[l + 1]; ++t) {
      const uint64_t i = members[t];
      const uint64_t id = ids ? ids[i] : n_old + i;
      nids.push_back(id);
      codes.insert(codes.end(), &newc[i * M], &newc[i * M] + M);
      if (host_.has_originals) {
        orig.insert(orig.end(), vectors + i * dim, vectors + (i + 1) * dim);
        ok.push_back(1);
      }
      n_tomb_ -= tomb_[l].erase(id);
    }
    offs[l + 1] = nids.size();
  }
  host_.offsets.swap(offs);
  host_.ids.swap(nids);
  host_.codes.swap(codes);
  if (host_.has_originals) {
    host_.originals.swap(orig);
    host_.orig_ok.swap(ok);
    // original_vectors.insert(id, vector) in input order (ivf_pq.rs:1769-1773):
    // the last vector given for an id becomes every entry's original for it
    std::unordered_map<uint64_t, uint64_t> last;
    for (uint64_t i = 0; i < n; ++i) last[ids ? ids[i] : n_old + i] = i;
    for (uint64_t p = 0; p < host_.ids.size(); ++p) {
      auto it = last.find(host_.ids[p]);
      if (it == last.end()) continue;
      std::memcpy(&host_.originals[p * dim], vectors + it->second * dim, 4 * (size_t)dim);
      host_.orig_ok[p] = 1;
    }
  }
  upload_lists();
}

void IvfPqIndex::search_filtered(const float* qs, uint64_t nq, uint32_t k, const uint64_t* allowed,
                                 uint64_t n_allowed, uint64_t* ids, float* dists, uint32_t* counts) {
  if (nq == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  const uint32_t kk = std::max<uint32_t>(k, 1);
  out_ids_.reserve(nq * kk);
  out_d_.reserve(nq * kk);
  out_cnt_.reserve(nq);
  // search_filtered probes take(nprobe): 0 lists when nprobe is 0 (:717-731);
  // no allowed id: no results (:700-703)
  uint32_t np = (uint32_t)std::min<uint64_t>(nprobe(), host_.nlist);
  if (n_allowed == 0) np = 0;
  q_.upload(qs, nq * host_.dim, stream_);
  const uint32_t* live = live_bitmap();
  const uint64_t N = host_.ids.size();
  if (np > 0) {
    std::vector<uint64_t> sorted(allowed, allowed + n_allowed);
    std::sort(sorted.begin(), sorted.end());
    allow_.upload(sorted.data(), sorted.size(), stream_);
    filt_.reserve(std::max<uint64_t>((N + 31) / 32, 1));
    FDB_HIP(launch_filter_bitmap(ids_.p, N, allow_.p, n_allowed, live, filt_.p, stream_));
  }
  run(q_.p, nq, k, np, kAdcGroups4, out_ids_.p, out_d_.p, out_cnt_.p, stream_, nullptr, nullptr,
      filt_.p, 4);
  if (k) {
    FDB_HIP(hipMemcpyAsync(ids, out_ids_.p, 8 * nq * k, hipMemcpyDeviceToHost, stream_));
    FDB_HIP(hipMemcpyAsync(dists, out_d_.p, 4 * nq * k, hipMemcpyDeviceToHost, stream_));
  }
  FDB_HIP(hipMemcpyAsync(counts, out_cnt_.p, 4 * nq, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
  throw_if_nan();
}

IvfPqIndex::~IvfPqIndex() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (auto& e : ev_)
    if (e) (void)hipEventDestroy(e);
  if (stream_) (void)hipStreamDestroy(stream_);
}

bool IvfPqIndex::set_lut_mode(int mode) {
  if (mode != 0 && mode != 1) return false;
  const bool shaped = (host_.M == 16 && host_.dsub == 8) || (host_.M == 32 && host_.dsub == 3);
  if (mode == 1 && !shaped) return false;
  lut_mode_.store(mode, std::memory_order_relaxed);
  return true;
}

void IvfPqIndex::enable_reranking(const float* v, uint64_t factor) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  const uint64_t N = host_.ids.size(), dim = host_.dim;
  host_.originals.assign(v, v + N * dim);
  host_.orig_ok.assign(N, 1);
  // the vectors are collected into a map by id (ivf_pq.rs:513-514): with
  // duplicate ids the last one in list order is every such entry's original
  std::unordered_map<uint64_t, uint64_t> last;
  last.reserve(N);
  bool dup = false;
  for (uint64_t p = 0; p < N; ++p) {
    auto r = last.emplace(host_.ids[p], p);
    if (!r.second) {
      r.first->second = p;
      dup = true;
    }
  }
  if (dup)
    for (uint64_t p = 0; p < N; ++p) {
      const uint64_t src = last[host_.ids[p]];
      if (src != p) std::memcpy(&host_.originals[p * dim], v + src * dim, 4 * (size_t)dim);
    }
  host_.has_originals = true;
  host_.rerank_factor = std::max<uint64_t>(factor, 1);
  upload_originals();
}

void IvfPqIndex::run(const float* d_qs, uint64_t nq, uint32_t k, uint32_t np, int order,
                     uint64_t* d_ids, float* d_dists, uint32_t* d_counts, hipStream_t s,
                     float* coarse_ms, float* scan_ms, const uint32_t* live, uint32_t fetch_mult) {
  if (nq == 0) return;
  if (k == 0 || np == 0) {
    hipLaunchKernelGGL(fill_empty_kernel, dim3(blocks_for(nq * std::max<uint32_t>(k, 1), 256)),
                       dim3(256), 0, s, nq, k, d_ids, d_dists, d_counts);
    FDB_HIP(hipGetLastError());
    if (coarse_ms) *coarse_ms = 0.0f;
    if (scan_ms) *scan_ms = 0.0f;
    return;
  }
  const bool rerank = host_.has_originals;
  const uint64_t factor = rerank ? host_.rerank_factor : 1;
  if (factor > 1024) throw Error(FDB_ERR_UNSUPPORTED, "candidates per query (k * rerank factor) above 1024");
  const uint64_t fetch = (uint64_t)k * factor * fetch_mult;
  if (fetch > 1024) throw Error(FDB_ERR_UNSUPPORTED, "candidates per query (k * rerank factor) above 1024");
  if (fetch == 0) {
    // a stored rerank_factor of 0 (from_serializable keeps it, ivf_pq.rs:1940)
    // keeps no candidate: every result is empty, as in the reference
    hipLaunchKernelGGL(fill_empty_kernel, dim3(blocks_for(nq * k, 256)), dim3(256), 0, s, nq, k, d_ids, d_dists,
                       d_counts);
    FDB_HIP(hipGetLastError());
    if (coarse_ms) *coarse_ms = 0.0f;
    if (scan_ms) *scan_ms = 0.0f;
    return;
  }
  // without reranking the kept candidates are truncated to k below
  const bool trunc = !rerank && fetch > k;
  if (np > 1024 && np < host_.nlist) throw Error(FDB_ERR_UNSUPPORTED, "nprobe above 1024");
  probes_.reserve(nq * np);
  const bool timed = coarse_ms || scan_ms;
  if (timed) FDB_HIP(hipEventRecord(ev_[0], s));
  if (np >= host_.nlist) {
    np = host_.nlist;
    hipLaunchKernelGGL(iota_probes_kernel, dim3(blocks_for(nq * np, 256)), dim3(256), 0, s, nq, np,
                       probes_.p);
    FDB_HIP(hipGetLastError());
    hipLaunchKernelGGL(nan_check_kernel, dim3(blocks_for(nq * host_.dim, 256)), dim3(256), 0, s,
                       d_qs, nq * host_.dim, err_.p);
    FDB_HIP(hipGetLastError());
  } else {
    coarse_.select(d_qs, nq, np, probes_.p, nullptr, err_.p, s);
  }
  if (timed) FDB_HIP(hipEventRecord(ev_[1], s));
  IvfPqScanArgs a{};
  a.queries = d_qs;
  a.nq = nq;
  a.dim = (int)host_.dim;
  a.M = (int)host_.M;
  a.dsub = (int)host_.dsub;
  a.probes = probes_.p;
  a.np = (int)np;
  a.nlist = (int)host_.nlist;
  a.centroids = centroids_.p;
  a.codebooks = codebooks_.p;
  a.list_off = off_.p;
  a.codes = codes_.p;
  a.ids = ids_.p;
  a.k = (int)fetch;
  a.order = order;
  a.lut_mode = lut_mode();
  a.cbnorm = cbnorm_.p;
  a.live = live;
  if (rerank || trunc) {
    cand_ids_.reserve(nq * fetch);
    cand_d_.reserve(nq * fetch);
    cand_pos_.reserve(nq * fetch);
    cand_cnt_.reserve(nq);
    a.out_ids = cand_ids_.p;
    a.out_dists = cand_d_.p;
    a.out_pos = cand_pos_.p;
    a.out_counts = cand_cnt_.p;
  } else {
    a.out_ids = d_ids;
    a.out_dists = d_dists;
    a.out_pos = nullptr;
    a.out_counts = d_counts;
  }
  // fp16 screening with exact rescoring (same results; fdb_ivfpq16.hpp):
  // plain exact-table batches over at least two lists
  const int smode = search_mode_.load(std::memory_order_relaxed);
  const uint64_t scanned = host_.nlist ? host_.ids.size() * np / host_.nlist : 0;
  bool screen = smode != 1 && !rerank && !trunc && live == nullptr && a.lut_mode == 0 && np >= 2 &&
                host_.M * host_.dsub <= 256 && (smode >= 2 || nq * scanned >= kPq16MinWork);
  if (screen && pq16_dirty_) {
    pq16_.build(codebooks_.p, codes_.p, off_.p, host_.offsets, host_.nlist, (int)host_.M, (int)host_.dsub, s);
    pq16_dirty_ = false;
  }
  screen = screen && pq16_.ok;
  path_ = screen ? 2 : 0;
  if (screen) {
    pq16s_.reset_stats(s);
    pq16s_.set_timing(timed);
    const uint64_t sl = std::min<uint64_t>(nq, Pq16Searcher::slice((int)k));
    const uint64_t D = host_.dim;
    for (uint64_t q0 = 0; q0 < nq; q0 += sl) {
      const uint64_t m = std::min<uint64_t>(sl, nq - q0);
      Pq16SearchArgs sa{};
      sa.tiles = smode == 3 ? 1 : -1;
      sa.queries = d_qs + q0 * D;
      sa.nq = m;
      sa.probes = probes_.p + q0 * np;
      sa.np = (int)np;
      sa.centroids = centroids_.p;
      sa.codebooks = codebooks_.p;
      sa.codes = codes_.p;
      sa.ids = ids_.p;
      sa.list_off = off_.p;
      sa.k = (int)k;
      sa.order = order;
      sa.out_ids = d_ids + q0 * k;
      sa.out_d = d_dists + q0 * k;
      sa.out_counts = d_counts + q0;
      pq16s_.search(pq16_, sa, s);
      // the queries screening did not settle: the exact scan
      IvfPqScanArgs af = a;
      af.queries = sa.queries;
      af.nq = m;
      af.probes = sa.probes;
      af.out_ids = sa.out_ids;
      af.out_dists = sa.out_d;
      af.out_counts = sa.out_counts;
      af.flags = pq16s_.flags();
      FDB_HIP(launch_ivfpq_scan(af, s));
    }
    if (timed) screen_kernel_ms_ = pq16s_.screen_ms();
    pq16s_.set_timing(false);
  } else {
    if (timed) screen_kernel_ms_ = 0.0f;
    FDB_HIP(launch_ivfpq_scan(a, s));
  }
  if (rerank)
    FDB_HIP(launch_rerank(d_qs, nq, (int)host_.dim, originals_.p, orig_all_ ? nullptr : orig_bits_.p, ids_.p,
                          cand_pos_.p, cand_cnt_.p, (uint32_t)fetch, k, d_ids, d_dists, d_counts, s));
  else if (trunc)
    FDB_HIP(launch_truncate(cand_ids_.p, cand_d_.p, cand_cnt_.p, nq, (uint32_t)fetch, k, d_ids, d_dists,
                            d_counts, s));
  if (timed) {
    FDB_HIP(hipEventRecord(ev_[2], s));
    FDB_HIP(hipEventSynchronize(ev_[2]));
    if (coarse_ms) FDB_HIP(hipEventElapsedTime(coarse_ms, ev_[0], ev_[1]));
    if (scan_ms) FDB_HIP(hipEventElapsedTime(scan_ms, ev_[1], ev_[2]));
  }
}

uint32_t IvfPqIndex::search(const float* q, uint32_t k, uint64_t* ids, float* dists) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  const uint32_t np = (uint32_t)std::min<uint64_t>(nprobe(), host_.nlist);  // 0 probes 0 lists
  q_.upload(q, host_.dim, stream_);
  const uint32_t kk = std::max<uint32_t>(k, 1);
  out_ids_.reserve(kk);
  out_d_.reserve(kk);
  out_cnt_.reserve(1);
  run(q_.p, 1, k, np, kAdcGroups4, out_ids_.p, out_d_.p, out_cnt_.p, stream_, nullptr, nullptr,
      live_bitmap());
  uint32_t cnt = 0;
  if (k) {
    FDB_HIP(hipMemcpyAsync(ids, out_ids_.p, 8 * (size_t)k, hipMemcpyDeviceToHost, stream_));
    FDB_HIP(hipMemcpyAsync(dists, out_d_.p, 4 * (size_t)k, hipMemcpyDeviceToHost, stream_));
  }
  FDB_HIP(hipMemcpyAsync(&cnt, out_cnt_.p, 4, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
  int flag = 0;
  FDB_HIP(hipMemcpy(&flag, err_.p, 4, hipMemcpyDeviceToHost));
  if (flag) {
    hipLaunchKernelGGL(clear_int_kernel, dim3(1), dim3(1), 0, stream_, err_.p);
    FDB_HIP(hipStreamSynchronize(stream_));
    throw Error(FDB_ERR_NAN, "NaN centroid distance (query contains NaN)");
  }
  return cnt;
}

void IvfPqIndex::batch_search(const float* qs, uint64_t nq, uint32_t k, uint64_t* ids,
                              float* dists, uint32_t* counts) {
  if (nq == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  // batch_search probes [..=nth]: at least one list (ivf_pq.rs:877-881)
  const uint32_t np = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(nprobe(), host_.nlist));
  q_.upload(qs, nq * host_.dim, stream_);
  const uint32_t kk = std::max<uint32_t>(k, 1);
  out_ids_.reserve(nq * kk);
  out_d_.reserve(nq * kk);
  out_cnt_.reserve(nq);
  run(q_.p, nq, k, np, kAdcLanes8, out_ids_.p, out_d_.p, out_cnt_.p, stream_, nullptr, nullptr,
      live_bitmap());
  if (k) {
    FDB_HIP(hipMemcpyAsync(ids, out_ids_.p, 8 * nq * k, hipMemcpyDeviceToHost, stream_));
    FDB_HIP(hipMemcpyAsync(dists, out_d_.p, 4 * nq * k, hipMemcpyDeviceToHost, stream_));
  }
  FDB_HIP(hipMemcpyAsync(counts, out_cnt_.p, 4 * nq, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
  int flag = 0;
  FDB_HIP(hipMemcpy(&flag, err_.p, 4, hipMemcpyDeviceToHost));
  if (flag) {
    hipLaunchKernelGGL(clear_int_kernel, dim3(1), dim3(1), 0, stream_, err_.p);
    FDB_HIP(hipStreamSynchronize(stream_));
    throw Error(FDB_ERR_NAN, "NaN centroid distance (a query contains NaN)");
  }
}

void IvfPqIndex::batch_search_device(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                                     float* d_dists, uint32_t* d_counts, hipStream_t s,
                                     float* coarse_ms, float* scan_ms) {
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, s ? s : stream_);
  const uint32_t np = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(nprobe(), host_.nlist));
  run(d_qs, nq, k, np, kAdcLanes8, d_ids, d_dists, d_counts, s ? s : stream_, coarse_ms, scan_ms,
      live_bitmap());
}

void IvfPqIndex::batch_search_device_noalloc(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                                             float* d_dists, uint32_t* d_counts, hipStream_t s, int32_t* probes,
                                             uint64_t cap) {
  std::lock_guard<std::mutex> g(mu_);
  const hipStream_t st = s ? s : stream_;
  OrderedOn on(order_, st);
  if (host_.has_originals)
    throw Error(FDB_ERR_UNSUPPORTED, "the no-allocation batch search serves indexes without reranking");
  if (n_tomb_ != 0)
    throw Error(FDB_ERR_UNSUPPORTED, "the no-allocation batch search serves indexes without tombstones");
  // batch_search probes [..=nth]: at least one list (ivf_pq.rs:877-881)
  const uint32_t np = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(nprobe(), host_.nlist));
  if (k > 1024) throw Error(FDB_ERR_UNSUPPORTED, "k above 1024");
  if (np > 1024 && np < host_.nlist) throw Error(FDB_ERR_UNSUPPORTED, "nprobe above 1024");
  if (nq * (uint64_t)np > cap)
    throw Error(FDB_ERR_UNSUPPORTED,
                "nq * nprobe above the no-allocation scratch (" + std::to_string(cap) + " probe entries)");
  if (nq == 0) return;
  if (k == 0) {
    hipLaunchKernelGGL(fill_empty_kernel, dim3(blocks_for(nq, 256)), dim3(256), 0, st, nq, k, d_ids, d_dists,
                       d_counts);
    FDB_HIP(hipGetLastError());
    return;
  }
  if (np >= host_.nlist) {
    hipLaunchKernelGGL(iota_probes_kernel, dim3(blocks_for(nq * np, 256)), dim3(256), 0, st, nq, np, probes);
    FDB_HIP(hipGetLastError());
    hipLaunchKernelGGL(nan_check_kernel, dim3(blocks_for(nq * host_.dim, 256)), dim3(256), 0, st, d_qs,
                       nq * host_.dim, err_.p);
    FDB_HIP(hipGetLastError());
  } else {
    coarse_.select_one_part(d_qs, nq, np, probes, err_.p, st);
  }
  IvfPqScanArgs a{};
  a.queries = d_qs;
  a.nq = nq;
  a.dim = (int)host_.dim;
  a.M = (int)host_.M;
  a.dsub = (int)host_.dsub;
  a.probes = probes;
  a.np = (int)np;
  a.nlist = (int)host_.nlist;
  a.centroids = centroids_.p;
  a.codebooks = codebooks_.p;
  a.list_off = off_.p;
  a.codes = codes_.p;
  a.ids = ids_.p;
  a.k = (int)k;
  a.order = kAdcLanes8;
  a.lut_mode = lut_mode();
  a.cbnorm = cbnorm_.p;
  a.live = nullptr;
  a.out_ids = d_ids;
  a.out_dists = d_dists;
  a.out_pos = nullptr;
  a.out_counts = d_counts;
  FDB_HIP(launch_ivfpq_scan(a, st));
  path_ = 0;
}

bool IvfPqIndex::sync(hipStream_t s) {
  std::lock_guard<std::mutex> g(mu_);
  FDB_HIP(hipStreamSynchronize(s ? s : stream_));
  int flag = 0;
  FDB_HIP(hipMemcpy(&flag, err_.p, 4, hipMemcpyDeviceToHost));
  if (flag) {
    hipLaunchKernelGGL(clear_int_kernel, dim3(1), dim3(1), 0, stream_, err_.p);
    FDB_HIP(hipStreamSynchronize(stream_));
  }
  return flag != 0;
}

void IvfPqIndex::probe(const float* qs, uint64_t nq, uint32_t nprobe, int32_t* lists,
                       float* dists) {
  if (nq == 0 || nprobe == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  if (nprobe > host_.nlist) throw Error(FDB_ERR_INVALID_ARGUMENT, "nprobe above nlist");
  if (nprobe > 1024) throw Error(FDB_ERR_UNSUPPORTED, "nprobe above 1024");
  q_.upload(qs, nq * host_.dim, stream_);
  probes_.reserve(nq * nprobe);
  probe_d_.reserve(nq * nprobe);
  coarse_.select(q_.p, nq, nprobe, probes_.p, probe_d_.p, err_.p, stream_);
  FDB_HIP(hipMemcpyAsync(lists, probes_.p, 4 * nq * nprobe, hipMemcpyDeviceToHost, stream_));
  if (dists)
    FDB_HIP(hipMemcpyAsync(dists, probe_d_.p, 4 * nq * nprobe, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
}

void IvfPqIndex::encode(const float* residuals, uint64_t nq, uint8_t* codes) {
  if (nq == 0) return;
  std::lock_guard<std::mutex> g(mu_);
  OrderedOn on(order_, stream_);
  // encode residuals directly: vectors = residuals, centroid rows = a zero row
  DevBuf<float> zero;
  std::vector<float> z(host_.dim, 0.0f);
  zero.upload(z.data(), z.size(), stream_);
  std::vector<uint64_t> rows(nq);
  for (uint64_t i = 0; i < nq; ++i) rows[i] = i;
  std::vector<int32_t> lists(nq, 0);
  DevBuf<uint64_t> d_rows;
  DevBuf<int32_t> d_lists;
  d_rows.upload(rows.data(), nq, stream_);
  d_lists.upload(lists.data(), nq, stream_);
  q_.upload(residuals, nq * host_.dim, stream_);
  codes_out_.reserve(nq * host_.M);
  FDB_HIP(launch_pq_encode(q_.p, d_rows.p, d_lists.p, nq, host_.dim, zero.p, codebooks_.p, host_.M,
                           host_.dsub, codes_out_.p, stream_));
  FDB_HIP(hipMemcpyAsync(codes, codes_out_.p, nq * host_.M, hipMemcpyDeviceToHost, stream_));
  FDB_HIP(hipStreamSynchronize(stream_));
}

// IVFPQIndex::build, ivf_pq.rs:374-506.  Sampling streams:
//   splitmix64_at(seed, 0)      training-sample shuffle (:383-396)
//   splitmix64_at(seed, 1)      coarse k-means initialisation (:398-400)
//   splitmix64_at(seed, 2)      PQ residual-sample shuffle (:422-446)
//   splitmix64_at(seed, 16 + m) PQ k-means initialisation of subspace m
IvfPqArtifacts IvfPqIndex::build(const float* vectors, const uint64_t* ids, uint64_t n,
                                 uint32_t dim, uint32_t nlist, uint32_t M, uint32_t metric,
                                 uint64_t seed) {
  if (n == 0 || dim == 0 || nlist == 0 || M == 0 || dim % M != 0)
    throw Error(FDB_ERR_INVALID_ARGUMENT, "build needs n, dim, nlist > 0 and M dividing dim");
  if (metric > 4) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown metric");
  if (n >= 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "more than 2^32-2 vectors");
  if (dim > 2048) throw Error(FDB_ERR_UNSUPPORTED, "dim above 2048");
  for (uint64_t i = 0; i < n * dim; ++i)
    if (std::isnan(vectors[i])) throw Error(FDB_ERR_NAN, "NaN in the vectors to index");
  const uint32_t dsub = dim / M;
  hipStream_t s;
  FDB_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  struct StreamGuard {
    hipStream_t s;
    ~StreamGuard() {
      (void)hipStreamSynchronize(s);
      (void)hipStreamDestroy(s);
    }
  } guard{s};
  auto row = [&](uint64_t i) { return vectors + i * (uint64_t)dim; };

  // 1. coarse centroids from a sample of at most 30k vectors
  const uint64_t ts = std::min<uint64_t>(n, 30000);
  std::vector<float> sample;
  if (n <= ts) {
    sample.assign(vectors, vectors + n * dim);
  } else {
    Stream rng(splitmix64_at(seed, 0));
    std::vector<uint64_t> idx(n);
    for (uint64_t i = 0; i < n; ++i) idx[i] = i;
    shuffle(rng, idx);
    sample.resize(ts * dim);
    for (uint64_t i = 0; i < ts; ++i) std::memcpy(&sample[i * dim], row(idx[i]), 4 * dim);
  }
  std::vector<float> cents = kmeans_gpu(sample.data(), ts, dim, nlist, 25, splitmix64_at(seed, 1), s);

  // 2. assign every vector to its nearest centroid
  DevBuf<float> d_vec, d_cent, d_centT;
  DevBuf<int32_t> d_assign;
  d_vec.upload(vectors, n * dim, s);
  d_cent.upload(cents.data(), cents.size(), s);
  d_centT.reserve((size_t)centT_ld(nlist) * dim);
  d_assign.reserve(n);
  FDB_HIP(launch_transpose_centroids(d_cent.p, nlist, dim, d_centT.p, s));
  FDB_HIP(launch_assign(d_vec.p, n, dim, d_centT.p, nlist, d_assign.p, s));
  std::vector<int32_t> assign(n);
  FDB_HIP(hipMemcpyAsync(assign.data(), d_assign.p, 4 * n, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  for (int32_t a : assign)
    if (a < 0 || a >= (int32_t)nlist) throw Error(FDB_ERR_NAN, "list assignment failed (NaN distance)");

  // 3. PQ codebooks from the residuals of a shuffled sample of <= 100k
  const uint64_t ps = std::min<uint64_t>(n, 100000);
  if (ps < 256) throw Error(FDB_ERR_INVALID_ARGUMENT, "PQ training needs at least 256 vectors");
  std::vector<float> resid(ps * dim);
  {
    Stream rng(splitmix64_at(seed, 2));
    std::vector<uint64_t> idx(n);
    for (uint64_t i = 0; i < n; ++i) idx[i] = i;
    shuffle(rng, idx);
    for (uint64_t t = 0; t < ps; ++t) {
      const float* v = row(idx[t]);
      const float* c = &cents[(size_t)assign[idx[t]] * dim];
      for (uint32_t j = 0; j < dim; ++j) resid[t * dim + j] = v[j] - c[j];
    }
  }
  std::vector<float> cb((size_t)M * 256 * dsub);
  std::vector<float> sub(ps * dsub);
  for (uint32_t m = 0; m < M; ++m) {
    for (uint64_t t = 0; t < ps; ++t) std::memcpy(&sub[t * dsub], &resid[t * dim + (size_t)m * dsub], 4 * dsub);
    std::vector<float> c = kmeans_gpu(sub.data(), ps, dsub, 256, 25, splitmix64_at(seed, 16 + m), s);
    std::memcpy(&cb[(size_t)m * 256 * dsub], c.data(), 4 * c.size());
  }

  // 4. lists in vector order, codes of the residuals
  IvfPqArtifacts a;
  a.nlist = nlist;
  a.dim = dim;
  a.M = M;
  a.dsub = dsub;
  a.metric = metric;
  a.nprobe = 1;
  a.centroids = std::move(cents);
  a.codebooks = std::move(cb);
  a.offsets.assign(nlist + 1, 0);
  for (uint64_t i = 0; i < n; ++i) a.offsets[assign[i] + 1]++;
  for (uint32_t l = 0; l < nlist; ++l) a.offsets[l + 1] += a.offsets[l];
  std::vector<uint64_t> fill(a.offsets.begin(), a.offsets.end() - 1);
  std::vector<uint64_t> rows(n);
  std::vector<int32_t> row_list(n);
  for (uint64_t i = 0; i < n; ++i) {
    const uint64_t p = fill[assign[i]]++;
    rows[p] = i;
    row_list[p] = assign[i];
  }
  a.ids.resize(n);
  for (uint64_t p = 0; p < n; ++p) a.ids[p] = ids ? ids[rows[p]] : rows[p];
  DevBuf<uint64_t> d_rows;
  DevBuf<int32_t> d_rl;
  DevBuf<float> d_cb;
  DevBuf<uint8_t> d_codes;
  d_rows.upload(rows.data(), n, s);
  d_rl.upload(row_list.data(), n, s);
  d_cb.upload(a.codebooks.data(), a.codebooks.size(), s);
  d_codes.reserve(n * M);
  FDB_HIP(launch_pq_encode(d_vec.p, d_rows.p, d_rl.p, n, dim, d_cent.p, d_cb.p, M, dsub, d_codes.p, s));
  a.codes.resize(n * M);
  FDB_HIP(hipMemcpyAsync(a.codes.data(), d_codes.p, n * M, hipMemcpyDeviceToHost, s));
  FDB_HIP(hipStreamSynchronize(s));
  return a;
}

}  // namespace fdb
