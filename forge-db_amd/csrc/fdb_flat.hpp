// Full-precision (uncompressed) search: BruteForceIndex (src/index/brute_force.rs)
// and IVFIndex (src/index/ivf.rs) on the GPU.
#pragma once

#include <atomic>
#include <mutex>
#include <vector>

#include "fdb_coarse16.hpp"
#include "fdb_host.hpp"
#include "fdb_ivfpq16.hpp"

namespace fdb {

// ---- kernels (fdb_flat.hip) ----------------------------------------------

// Row-major rows [n][dim] -> dim-major, rows permuted like centT:
// out[prow(d) * ld + r] (ld >= n, multiple of 4; padding is zero).
hipError_t launch_transpose_rows(const float* rows, uint64_t n, int dim, uint64_t ld, float* out,
                                 hipStream_t s);
// Reference-order sum of squares (the norms of cosine_distance_avx2,
// simd.rs:466-507) of n row-major vectors.
hipError_t launch_row_norms(const float* rows, uint64_t n, int dim, float* out, hipStream_t s);

// Brute-force partial top-k: queries [nq][dim]; data [dim][ld] permuted;
// rows [0, n) cut into chunks of chunk_rows; writes per (query, chunk) the k
// smallest (distance, row) pairs into part [nq][nchunks][k].
struct FlatTopkArgs {
  const float* queries;
  uint64_t nq;
  int dim;
  const float* dataT;
  uint64_t ld, n;
  const float* row_norm;  // cosine only
  const float* q_norm;    // cosine only
  uint64_t chunk_rows;
  uint32_t nchunks;
  int metric;
  int k;
  float* part_d;
  uint32_t* part_key;
  const int* flags;  // nullable: [nq]; tiles without a nonzero flag return at once
};
hipError_t launch_flat_topk(const FlatTopkArgs& a, hipStream_t s);

// Merge [nq][nparts][k] partial lists into [nq][k] ascending (ties: smaller
// key), keys mapped to ids through ids (nullable: keys are the ids).
// flags (nullable): only queries with a nonzero flag are written.
hipError_t launch_merge_parts(const float* part_d, const uint32_t* part_key, uint64_t nq,
                              uint32_t nparts, int k, const uint64_t* ids, uint64_t* out_ids,
                              float* out_d, uint32_t* out_counts, hipStream_t s,
                              const int* flags = nullptr);

// MFMA screening (dot, cosine, squared L2): per (32-query tile, row chunk)
// the K' = kp smallest screening values; grid x = query tiles, y = chunks.
struct ScreenArgs {
  const float* queries;  // [nq][dim]
  uint64_t nq;
  int dim;  // a multiple of 4, <= 512
  const float* dataT;
  uint64_t ld, n;
  const float* row_norm;  // [n] reference-order squared norms
  const float* q_norm;    // [nq]
  uint64_t chunk_rows;    // a multiple of 256
  uint32_t nchunks;
  int metric;
  int kp;  // 64 or 128
  float* part_d;
  uint32_t* part_key;
};
hipError_t launch_mfma_screen(const ScreenArgs& a, hipStream_t s);

// Exact rescoring of screened candidates ([nq][kp], ascending, as merged):
// writes the k smallest exact results, flags [nq] (1 = the candidates may
// miss a top-k row) and adds the number of flagged queries to *fallbacks.
// bkind selects the check:
//   kBoundF32:   fp32 screening, the K'-th candidate value minus screen_eps
//                bounds every other row;
//   kBoundH16:   fp16 brute-force screening (screen16_eps); abound[q] bounds
//                the rows outside, and fewer than min(k, n) candidates is a
//                miss;
//   kBoundIvf16: fp16 IVF screening (ivf16_bound; xmag, xexp); abound[q]
//                (+inf: every scanned row is a candidate) against the bound
//                of the k-th value.
// A query with cand_counts = kForceExact is flagged.
constexpr uint32_t kForceExact = 0xFFFFFFFFu;
enum { kBoundF32 = 0, kBoundH16 = 1, kBoundIvf16 = 2 };
struct RescoreArgs {
  const float* queries;
  int dim;
  const float* rows;  // [n][dim] row-major
  const float* row_norm;
  const float* q_norm;
  float rnmax;  // the largest row norm (squared)
  const uint64_t* cand_keys;
  const float* cand_d;
  const uint32_t* cand_counts;
  int kp;
  int metric;
  int k;
  const uint64_t* ids;
  uint64_t* out_ids;
  float* out_d;
  uint32_t* out_counts;
  int* flags;
  uint32_t* fallbacks;
  const float* abound;
  int bkind;
  uint64_t n;
  float xmag;  // kBoundIvf16: max |x|_2 (max |x|_1 for Manhattan) over the rows
  int xexp;    // kBoundIvf16: the rows' fp16 scale exponent
};
hipError_t launch_rescore(const RescoreArgs& a, uint64_t nq, hipStream_t s);

// IVF-flat scan: per query, probes [nq][np] lists of list-blocked data
// (list p: block [dim][lld_p] at boff[p] floats, rows start at row_off[p]).
struct IvfFlatScanArgs {
  const float* queries;
  uint64_t nq;
  int dim;
  const int32_t* probes;
  int np;
  int nlist;
  const float* data;         // list blocks
  const uint64_t* boff;      // [nlist] float offset of each list block
  const uint32_t* row_off;   // [nlist+1] row offsets (list order)
  const float* row_norm;     // cosine: [N] in list order
  const float* q_norm;       // cosine: [nq]
  const uint64_t* ids;       // [N] list order
  int metric;
  int k;
  uint64_t* out_ids;
  float* out_d;
  uint32_t* out_counts;
  const int* flags;  // nullable: [nq]; queries with a zero flag return at once
};
hipError_t launch_ivf_flat_scan(const IvfFlatScanArgs& a, hipStream_t s);

// The lists of an IVF index in half precision for screening (fdb_ivf16.hip):
// per list a block [dim2][lld] of 32-bit words, word (j, r) the pair
// (x_2j, x_2j+1) * 2^xexp of row r as two halves (lld = |L_p| rounded up to
// 4; an odd dim is padded with a zero), and the rows' largest L2 and L1
// norms.  ok = false when the rows are not finite or their scale is out of
// reach.
struct Ivf16Lists {
  bool ok = false;
  int dim_ = 0, dim2 = 0, xexp = 0;
  float xnorm2_max = 0.0f, xnorm1_max = 0.0f;
  // d_rows [N][dim] row-major in list order; offsets [nlist+1]
  void build(const float* d_rows, const std::vector<uint64_t>& offsets, uint32_t nlist, int dim,
             const uint32_t* d_row_off, hipStream_t s);
  // the kp (64 or 128) smallest screening values per query over its probed
  // lists: cand_d/cand_k [nq][kp] (list positions), cand_c [nq] (kForceExact
  // when the query does not fit fp16), abound [nq] (the kp-th value, +inf when
  // every scanned row is a candidate); l1: Manhattan, else squared L2
  hipError_t screen(const float* d_qs, uint64_t nq, const int32_t* probes, uint32_t np, uint32_t nlist,
                    const uint32_t* d_row_off, bool l1, int kp, float* cand_d, uint64_t* cand_k, uint32_t* cand_c,
                    float* abound, hipStream_t s) const;

 private:
  DevBuf<uint32_t> data_, stats_;
  DevBuf<uint64_t> boff_;
};

// ---- exact and screened top-k over a row set ------------------------------

// A row set resident on the device, as the flat searches read it.
struct FlatRows {
  const float* dataT;     // [dim][ld] dimension rows permuted (launch_transpose_rows)
  uint64_t ld, n;
  int dim;
  const float* rows;      // [n][dim] row-major (rescoring of screened candidates)
  const float* row_norm;  // [n] reference-order squared norms
  float rnmax;            // the largest of them
  const uint64_t* ids;    // nullable: results carry row indices
};

// The rows of a FlatRows as the fp16 screening reads them: 32-row blocks of
// MFMA A operands (kb k-steps of 16 dimensions, zero-padded), scaled by
// 2^xexp (cosine: each row divided by its norm first), and for Euclidean the
// squared norms zero-padded to whole blocks.  ok = false when the rows do
// not fit fp16 (non-finite values, zero-norm rows for cosine, a dimension
// above 512 or not a multiple of 4, Manhattan).
int h16_ksteps(int dim);
struct H16Rows {
  bool ok = false;
  uint64_t n_ = 0, nblk = 0;
  int dim_ = 0, kb = 0, xexp = 0;
  float rnmin = 0.0f;  // cosine: the smallest squared row norm
  void build(const float* rows, const float* row_norm, uint64_t n, int dim, int metric, hipStream_t s);
  const uint16_t* x16() const { return x16_.p; }
  const float* rn16() const { return rn16_.p; }

 private:
  DevBuf<uint16_t> x16_;
  DevBuf<float> rn16_;
  DevBuf<uint32_t> stats_;
};

// The k smallest (distance, row) per query over a FlatRows, by the exact VALU
// scan or by MFMA screening + exact rescoring (same results).  Owns its
// scratch; one user at a time.
class FlatSearcher {
 public:
  // whether screening serves (metric, dim, k)
  static bool screenable(int metric, int dim, uint32_t k);
  static bool screenable16(const H16Rows& h, int metric, uint32_t k);
  // q_norm: [nq] reference-order query norms (cosine and screening)
  void exact(const FlatRows& x, int metric, const float* d_qs, const float* q_norm, uint64_t nq,
             uint32_t k, uint64_t* ids, float* d, uint32_t* c, hipStream_t s, const int* flags = nullptr);
  void screen(const FlatRows& x, int metric, const float* d_qs, const float* q_norm, uint64_t nq,
              uint32_t k, uint64_t* ids, float* d, uint32_t* c, hipStream_t s);
  // fp16 screening (fdb_screen16.hip) over the same rows prepared as h
  void screen16(const FlatRows& x, const H16Rows& h, int metric, const float* d_qs, const float* q_norm,
                uint64_t nq, uint32_t k, uint64_t* ids, float* d, uint32_t* c, hipStream_t s);
  // device counter: queries of the last screen() rescanned exactly
  const uint32_t* fallbacks() const { return fallbacks_.p; }

 private:
  DevBuf<float> part_d_, cand_d_, tau_, abound_;
  DevBuf<uint32_t> part_k_, cand_c_, fallbacks_, count_;
  DevBuf<uint64_t> cand_k_;
  DevBuf<int> flags_, qexp_, force_;
  DevBuf<uint16_t> q16_;
  DevBuf<uint2> buf_;
};

// ---- coarse quantizer ---------------------------------------------------------

// Selection of the nprobe nearest of nlist centroids (squared L2 in the
// reference's order, ascending by (distance, list id)): the exact VALU kernel
// (launch_coarse_select) or fp16 matrix-core screening with exact rescoring
// (Coarse16, fdb_coarse16.hpp), which returns the same lists and distances.
class CoarseQuantizer {
 public:
  // centroids [nlist][dim] and their transposed copy (launch_transpose_centroids),
  // both device-resident and owned by the caller; builds the fp16 blocks
  void init(const float* centroids, const float* centT, uint32_t nlist, uint32_t dim, hipStream_t s);
  // 0 = automatic (screening where it applies: nprobe <= 64 and nlist >=
  // 256), 1 = exact kernel only, 2 = screening where it applies
  void set_mode(int m) { mode_ = m; }
  // probes [nq][np] (np <= nlist, <= 1024); dists [nq][np] nullable; a NaN
  // distance ORs 1 into *err
  void select(const float* d_qs, uint64_t nq, uint32_t np, int32_t* probes, float* dists, int* err,
              hipStream_t s);
  // The exact kernel in one part (the same probes): uses no device memory
  // beyond probes and err.
  void select_one_part(const float* d_qs, uint64_t nq, uint32_t np, int32_t* probes, int* err,
                       hipStream_t s) const;

 private:
  const float* cent_ = nullptr;
  const float* centT_ = nullptr;
  uint32_t nlist_ = 0, dim_ = 0;
  int mode_ = 0;
  Coarse16 c16_;
  DevBuf<int> flags_;
  DevBuf<float> part_d_;
  DevBuf<uint32_t> part_k_;
};

// ---- BruteForceIndex ------------------------------------------------------

class BruteForceIndex {
 public:
  // BruteForceIndex::new (brute_force.rs:67): empty, dimension set by the
  // first add.
  explicit BruteForceIndex(uint32_t metric);
  ~BruteForceIndex();
  uint64_t size() const { return h_ids_.size(); }
  uint32_t dim() const { return h_ids_.empty() ? 0 : dim_; }
  uint32_t metric() const { return metric_; }
  const std::vector<float>& rows() const { return h_rows_; }
  const std::vector<uint64_t>& ids() const { return h_ids_; }

  // add (brute_force.rs:75 / MutableVectorIndex::add :254-265): appends n
  // rows [n][dim] with ids (nullable: ids continue from size()).
  void add(const float* rows, const uint64_t* ids, uint64_t n, uint32_t dim);
  // MutableVectorIndex::remove (:267-274): the first row with this id is
  // replaced by the last row (VectorStore::swap_remove, vector.rs:256-270).
  bool remove(uint64_t id);

  // search / search_parallel (brute_force.rs:162-214): one query
  uint32_t search(const float* q, uint32_t k, uint64_t* ids, float* dists);
  // batch_search (brute_force.rs:220-225)
  void batch_search(const float* qs, uint64_t nq, uint32_t k, uint64_t* ids, float* dists,
                    uint32_t* counts);
  void batch_search_device(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                           float* d_dists, uint32_t* d_counts, hipStream_t s, float* ms = nullptr);

  // 0 = automatic (MFMA screening where it applies), 1 = exact VALU scan
  // only, 2 = screening where it applies, 3 = screening with the fp32
  // product only (modes 0 and 2 take the fp16 product where the rows fit it)
  void set_screen_mode(int m) { screen_mode_ = m; }
  int screen_mode() const { return screen_mode_; }
  // queries of the last search that the screening check sent to the exact
  // scan (waits for the stream s, null: own stream)
  uint64_t last_fallbacks(hipStream_t s);
  // how the last search ran: 0 exact scan, 1 fp32 screening, 2 fp16 screening
  int last_path() {
    std::lock_guard<std::mutex> g(mu_);
    return path_;
  }

 private:
  void sync_device();  // re-uploads the rows after add/remove (caller holds mu_)
  void run(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists,
           uint32_t* d_counts, hipStream_t s);
  bool screen_applies(uint64_t nq, uint32_t k) const;
  FlatRows flat_rows() const;

  uint32_t dim_ = 0, metric_;
  std::vector<float> h_rows_;
  std::vector<uint64_t> h_ids_;
  bool dirty_ = false;
  uint64_t n_dev_ = 0;  // rows resident on the device
  hipStream_t stream_ = nullptr;
  std::mutex mu_;
  StreamOrder order_;  // calls on different streams share the scratch below
  DevBuf<float> dataT_, row_norm_, rows_;
  DevBuf<uint64_t> ids_;
  uint64_t ld_ = 0;
  float rnmax_ = 0.0f;
  H16Rows h16_;
  int screen_mode_ = 0;
  int path_ = 0;  // the last search: 0 exact scan, 1 fp32 screening, 2 fp16 screening
  // scratch
  FlatSearcher srch_;
  DevBuf<float> q_, qn_, out_d_;
  DevBuf<uint32_t> out_c_;
  DevBuf<uint64_t> out_i_;
  hipEvent_t ev_[2] = {nullptr, nullptr};
};

// ---- IVFIndex ---------------------------------------------------------------

class IvfFlatIndex {
 public:
  // centroids [nlist][dim]; lists in CSR over rows [N][dim] (list order), ids
  IvfFlatIndex(const float* centroids, uint32_t nlist, uint32_t dim, const uint64_t* offsets,
               const uint64_t* ids, const float* rows, uint32_t metric);
  ~IvfFlatIndex();
  // IVFIndex::build (ivf.rs:91-119) on the GPU with a seeded k-means
  static IvfFlatIndex* build(const float* vectors, const uint64_t* ids, uint64_t n, uint32_t dim,
                             uint32_t nlist, uint32_t metric, uint32_t max_iters, uint64_t seed);

  uint32_t nlist() const { return nlist_; }
  uint32_t metric() const { return metric_; }
  // coarse selection strategy (CoarseQuantizer::set_mode)
  void set_coarse_mode(int m) {
    std::lock_guard<std::mutex> g(mu_);
    coarse_.set_mode(m);
  }
  // scan strategy: 0 = automatic (for Euclidean and squared Euclidean,
  // batches of at least 2^26 (query, row) pairs screen the lists on the
  // matrix cores, list by list; else fp16 screening per query + exact
  // rescoring for Euclidean, squared Euclidean and Manhattan when k <= 112
  // and dim is a multiple of 4, <= 512), 1 = exact scan only, 2 = the
  // list screening wherever it applies (Euclidean and squared Euclidean,
  // dim <= 256, nprobe >= 2), else as 0; same results
  void set_search_mode(int m) {
    std::lock_guard<std::mutex> g(mu_);
    search_mode_ = m;
  }
  // queries of the last search rescanned exactly after screening (waits for s)
  uint64_t last_fallbacks(hipStream_t s);
  // how the last search ran: 0 exact scan, 2 fp16 screening per query, 3
  // list screening on the matrix cores
  int last_path() {
    std::lock_guard<std::mutex> g(mu_);
    return path_;
  }
  // duration of the list screening's threshold kernel in the last timed
  // batch (0 when it did not take list screening)
  float last_screen_kernel_ms() {
    std::lock_guard<std::mutex> g(mu_);
    return screen_kernel_ms_;
  }
  uint32_t dim() const { return dim_; }
  uint64_t size() const { return h_ids_.size(); }
  void set_nprobe(uint64_t np) { nprobe_.store(np < nlist_ ? np : nlist_, std::memory_order_relaxed); }
  uint64_t nprobe() const { return nprobe_.load(std::memory_order_relaxed); }
  void export_to(float* centroids, uint64_t* offsets, uint64_t* ids, float* rows) const;

  // search (ivf.rs:162-216) and batch_search (ivf.rs:292-297)
  void batch_search(const float* qs, uint64_t nq, uint32_t k, uint64_t* ids, float* dists,
                    uint32_t* counts);
  void batch_search_device(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids,
                           float* d_dists, uint32_t* d_counts, hipStream_t s, float* coarse_ms = nullptr,
                           float* scan_ms = nullptr);
  // the nprobe nearest lists per query, ascending by (squared L2, list id)
  // (the stable sort of ivf.rs:164-177)
  void probe(const float* qs, uint64_t nq, uint32_t nprobe, int32_t* lists);
  // waits for s (null: own stream); true if a device search saw a NaN since
  // the last sync (the flag is cleared)
  bool sync(hipStream_t s);

 private:
  void run(const float* d_qs, uint64_t nq, uint32_t k, uint64_t* d_ids, float* d_dists,
           uint32_t* d_counts, hipStream_t s, float* coarse_ms, float* scan_ms);

  uint32_t nlist_, dim_, metric_;
  std::atomic<uint64_t> nprobe_{1};
  std::vector<float> h_centroids_, h_rows_;
  std::vector<uint64_t> h_offsets_, h_ids_;
  hipStream_t stream_ = nullptr;
  std::mutex mu_;
  StreamOrder order_;  // calls on different streams share the scratch below
  DevBuf<float> centT_, cent_, data_, row_norm_;
  DevBuf<float> rowsl_;  // [N][dim] row-major, list order (rescoring)
  Ivf16Lists l16_;
  Pq16Lists p16_;        // the rows as matrix-core blocks (built on first use)
  bool p16_tried_ = false;
  Pq16Searcher p16s_;
  static constexpr uint64_t kListScreenMinWork = 1ull << 26;  // (query, row) pairs
  float screen_kernel_ms_ = 0.0f;
  int search_mode_ = 0, path_ = 0;
  DevBuf<float> cand_d_, abound_;
  DevBuf<uint64_t> cand_k_;
  DevBuf<uint32_t> cand_c_, fallbacks_;
  DevBuf<int> flags_;
  CoarseQuantizer coarse_;
  DevBuf<uint64_t> boff_, ids_;
  DevBuf<uint32_t> row_off_;
  DevBuf<float> q_, qn_, out_d_;
  DevBuf<int32_t> probes_;
  DevBuf<uint64_t> out_i_;
  DevBuf<uint32_t> out_c_;
  DevBuf<int> err_;
  hipEvent_t ev_[3] = {nullptr, nullptr, nullptr};
};

}  // namespace fdb
