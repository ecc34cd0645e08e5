// IVF-PQ index resident on one GPU: the host-side mirror of IVFPQIndex
// (src/index/ivf_pq.rs:343-359) around the HIP kernels.
#pragma once

#include <atomic>
#include <mutex>
#include <unordered_set>
#include <vector>

#include "fdb_flat.hpp"
#include "fdb_format.hpp"
#include "fdb_host.hpp"
#include "fdb_ivfpq16.hpp"

namespace fdb {

class IvfPqIndex {
 public:
  // Takes the artifacts (validated by the caller) and uploads them.
  explicit IvfPqIndex(IvfPqArtifacts&& art);
  ~IvfPqIndex();

  // IVFPQIndex::build, ivf_pq.rs:374-506, on the GPU with seeded sampling.
  static IvfPqArtifacts build(const float* vectors, const uint64_t* ids, uint64_t n, uint32_t dim,
                              uint32_t nlist, uint32_t M, uint32_t metric, uint64_t seed);

  const IvfPqArtifacts& artifacts() const { return host_; }
  uint32_t nlist() const { return host_.nlist; }
  uint32_t dim() const { return host_.dim; }
  uint64_t size() const { return host_.ids.size(); }

  void set_nprobe(uint64_t np) { nprobe_.store(np < host_.nlist ? np : host_.nlist, std::memory_order_relaxed); }
  uint64_t nprobe() const { return nprobe_.load(std::memory_order_relaxed); }

  // 0 = exact LUTs (the reference's rounding), 1 = fast LUTs; returns false
  // when the index shape has no fast kernel
  bool set_lut_mode(int mode);
  int lut_mode() const { return lut_mode_.load(std::memory_order_relaxed); }
  // coarse selection strategy (CoarseQuantizer::set_mode)
  void set_coarse_mode(int m) {
    std::lock_guard<std::mutex> g(mu_);
    coarse_.set_mode(m);
  }

  void enable_reranking(const float* vectors_list_order, uint64_t factor);

  // 0 = automatic (fp16 screening with exact rescoring for large plain
  // batches, fdb_ivfpq16.hpp), 1 = exact scan only, 2 = screening wherever
  // it applies, 3 = as 2 with size-sorted tiles from per-XCD counters
  // whatever the index size; the results are the same
  bool set_search_mode(int m) {
    if (m < 0 || m > 3) return false;
    search_mode_.store(m, std::memory_order_relaxed);
    return true;
  }
  // the last batch: 2 = screened, 0 = exact scan; queries it rescanned
  // exactly and candidates it rescored
  int last_search_path() {
    std::lock_guard<std::mutex> g(mu_);
    return path_;
  }
  void last_screen_stats(uint64_t& fallbacks, uint64_t& candidates, hipStream_t s);
  // duration of the threshold screening kernel in the last timed batch (0
  // when it took the table scan)
  float last_screen_kernel_ms() {
    std::lock_guard<std::mutex> g(mu_);
    return screen_kernel_ms_;
  }

  // single query with search() semantics; returns count
  uint32_t search(const float* q, uint32_t k, uint64_t* ids, float* dists);
  // batch_search over host buffers
  void batch_search(const float* qs, uint64_t nq, uint32_t k, uint64_t* ids, float* dists,
                    uint32_t* counts);
  // batch_search over device buffers, enqueue only
  void batch_search_device(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                           float* d_dists, uint32_t* d_counts, hipStream_t stream,
                           float* coarse_ms = nullptr, float* scan_ms = nullptr);
  // returns true when a NaN was seen since the last call
  bool sync(hipStream_t stream);
  // batch_search_device without device allocation: the table scan, with
  // the [nq][nprobe] probe lists in `probes` (cap entries; the caller's
  // static scratch).  Plain indexes only (no reranking, no tombstones).
  void batch_search_device_noalloc(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists,
                                   uint32_t* d_counts, hipStream_t stream, int32_t* probes, uint64_t cap);
  void probe(const float* qs, uint64_t nq, uint32_t nprobe, int32_t* lists, float* dists);
  void encode(const float* residuals, uint64_t nq, uint8_t* codes);

  // search_filtered (ivf_pq.rs:692-831) for each of nq queries: only list
  // positions whose id is in allowed (n_allowed ids, any order) and not
  // tombstoned are scanned, with 4 * fetch_k candidates kept per query.
  void search_filtered(const float* qs, uint64_t nq, uint32_t k, const uint64_t* allowed,
                       uint64_t n_allowed, uint64_t* ids, float* dists, uint32_t* counts);
  // delete (ivf_pq.rs:1786-1804): tombstones id in the first list holding it
  // untombstoned; false when there is none.
  bool remove(uint64_t id);
  // insert_batch (ivf_pq.rs:1731-1776): nearest list, residual encoded with
  // the codebooks, appended in input order; the id leaves that list's
  // tombstones.  With reranking on, the vectors join the originals.
  void insert(const float* vectors, const uint64_t* ids, uint64_t n);
  // compact (ivf_pq.rs:1828-1851): drops tombstoned entries.
  void compact();
  // num_tombstones (:1807-1812); len() = entries - tombstones (:1088-1094)
  uint64_t num_tombstones() const { return n_tomb_; }
  uint64_t live_len() const { return host_.ids.size() - n_tomb_; }

  hipStream_t stream() const { return stream_; }

 private:
  // the device pipeline: coarse selection, fused scan, optional rerank.
  // live: bitmap of scannable list positions (nullable); fetch_mult scales
  // the candidates kept per query before reranking/truncation.
  void run(const float* d_qs, uint64_t nq, uint32_t k, uint32_t np, int order, uint64_t* d_ids,
           float* d_dists, uint32_t* d_counts, hipStream_t s, float* coarse_ms, float* scan_ms,
           const uint32_t* live = nullptr, uint32_t fetch_mult = 1);
  // tombstone bitmap for the scan, rebuilt after changes (caller holds mu_);
  // null when nothing is tombstoned
  const uint32_t* live_bitmap();
  // re-uploads ids, codes, offsets and originals after the lists changed
  void upload_lists();
  // uploads the originals and, when some entry has none, their bitmap
  void upload_originals();
  // every entry holding id gets original v (null: none)
  void set_original(uint64_t id, const float* v);
  void throw_if_nan();

  IvfPqArtifacts host_;
  std::atomic<uint64_t> nprobe_{1};
  std::atomic<int> lut_mode_{0};
  std::atomic<int> search_mode_{0};
  // automatic screening from this many scanned codes per batch
  static constexpr uint64_t kPq16MinWork = 1ull << 26;
  hipStream_t stream_ = nullptr;
  std::mutex mu_;
  StreamOrder order_;  // calls on different streams share the scratch below

  DevBuf<float> centroids_, centT_, codebooks_, cbnorm_, originals_;
  // one bit per list entry: it has an original vector (uploaded only when
  // some entry has none)
  DevBuf<uint32_t> orig_bits_;
  bool orig_all_ = true;
  CoarseQuantizer coarse_;
  DevBuf<uint32_t> off_;
  DevBuf<uint8_t> codes_;
  DevBuf<uint64_t> ids_;

  // tombstones per list (PartitionData::tombstones, ivf_pq.rs:190) and the
  // bitmap of untombstoned list positions
  std::vector<std::unordered_set<uint64_t>> tomb_;
  uint64_t n_tomb_ = 0;
  bool live_dirty_ = false;
  DevBuf<uint32_t> live_, filt_;
  DevBuf<uint64_t> allow_;

  // per-call scratch, guarded by mu_
  DevBuf<float> q_, probe_d_, cand_d_, out_d_;
  DevBuf<int32_t> probes_;
  DevBuf<uint64_t> cand_ids_, out_ids_;
  DevBuf<uint32_t> cand_pos_, cand_cnt_, out_cnt_;
  DevBuf<int> err_;
  DevBuf<uint8_t> codes_out_;
  hipEvent_t ev_[3] = {nullptr, nullptr, nullptr};

  // screening: the decoded lists (rebuilt after the lists change) and its
  // scratch
  Pq16Lists pq16_;
  bool pq16_dirty_ = true;
  Pq16Searcher pq16s_;
  int path_ = 0;
  float screen_kernel_ms_ = 0.0f;
};

// The current device's no-allocation scratch (probe lists; cap entries).
int32_t* noalloc_scratch(uint64_t& cap);

// Seeded k-means over n host rows [n][dim] (KMeans::fit_raw, kmeans.rs:87-193):
// k centroids [k][dim] after at most max_iters Lloyd steps on the GPU.
std::vector<float> kmeans_gpu(const float* h_points, uint64_t n, int dim, int k, int max_iters,
                              uint64_t seed, hipStream_t s);

}  // namespace fdb
