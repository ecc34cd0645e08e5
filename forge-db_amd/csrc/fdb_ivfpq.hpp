// IVF-PQ index resident on one GPU: the host-side mirror of IVFPQIndex
// (src/index/ivf_pq.rs:343-359) around the HIP kernels.
#pragma once

#include <atomic>
#include <mutex>

#include "fdb_format.hpp"
#include "fdb_host.hpp"

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

  void enable_reranking(const float* vectors_list_order, uint64_t factor);

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
  void probe(const float* qs, uint64_t nq, uint32_t nprobe, int32_t* lists, float* dists);
  void encode(const float* residuals, uint64_t nq, uint8_t* codes);

  hipStream_t stream() const { return stream_; }

 private:
  // the device pipeline: coarse selection, fused scan, optional rerank
  void run(const float* d_qs, uint64_t nq, uint32_t k, uint32_t np, int order, uint64_t* d_ids,
           float* d_dists, uint32_t* d_counts, hipStream_t s, float* coarse_ms, float* scan_ms);

  IvfPqArtifacts host_;
  std::atomic<uint64_t> nprobe_{1};
  std::atomic<int> lut_mode_{0};
  hipStream_t stream_ = nullptr;
  std::mutex mu_;

  DevBuf<float> centroids_, centT_, codebooks_, cbnorm_, originals_;
  DevBuf<uint32_t> off_;
  DevBuf<uint8_t> codes_;
  DevBuf<uint64_t> ids_;

  // per-call scratch, guarded by mu_
  DevBuf<float> q_, probe_d_, cand_d_, out_d_;
  DevBuf<int32_t> probes_;
  DevBuf<uint64_t> cand_ids_, out_ids_;
  DevBuf<uint32_t> cand_pos_, cand_cnt_, out_cnt_;
  DevBuf<int> err_;
  DevBuf<uint8_t> codes_out_;
  hipEvent_t ev_[3] = {nullptr, nullptr, nullptr};
};

// Seeded k-means over n host rows [n][dim] (KMeans::fit_raw, kmeans.rs:87-193):
// k centroids [k][dim] after at most max_iters Lloyd steps on the GPU.
std::vector<float> kmeans_gpu(const float* h_points, uint64_t n, int dim, int k, int max_iters,
                              uint64_t seed, hipStream_t s);

}  // namespace fdb
