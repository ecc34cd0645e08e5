// IVF-PQ screening on the matrix cores (fdb_ivfpq16.hip).
//
// The reference scores every code of the probed lists through per-list
// distance tables (src/pq.rs:149-189, :318-485; src/index/ivf_pq.rs:590-677).
// Here a batch is searched in three steps whose result equals the exact
// scan's, ties included:
//   the screened distance of a code x in list p is
//   s = |r|^2 + |x^|^2 - 2<r, x^> with r = q - c_p and x^ its decoded residual
//   (the concatenated codewords), <r, x^> from fp16 products on the matrix
//   cores; eps_qp bounds |s - d| for the reference's fp32 table distance d
//   (pq16_eps);
//   1. over the query's first probed lists holding at least k codes (at
//      most cap_first(k) values kept), d_k = (k-th smallest s) + max eps: at least
//      k codes have d <= d_k, so the final k-th distance is <= d_k;
//   2. over every probed list, the codes with s <= d_k + eps_qp become
//      candidates;
//   3. the candidates' distances are recomputed in the reference's order
//      and the k smallest kept.
// A code left out has d >= s - eps_qp > d_k >= the final k-th distance, so it
// cannot be in the result.  Queries whose candidates overflow, or whose
// residuals do not fit fp16, are rescanned exactly.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <utility>
#include <vector>

#include "fdb_host.hpp"

namespace fdb {

// Decoded residuals of every code in half precision, blocked for
// v_mfma_f32_32x32x16_f16: list p owns blocks [bo[p], bo[p+1]) of 32 codes
// (the last one padded with zeros); block b, k-chunk kc (16 dimensions; the
// dimension is padded to a multiple of 16) is 64 lanes x 8 halves, lane l
// holding code l%32, dimensions 16kc + 8(l/32) .. +7, scaled by 2^xexp.
// xnb [blocks*32]: |x^|^2 of each code in fp32 (0 for padding); xmax2
// [nlist]: bits of the list's largest |x^|^2.
struct Pq16Lists {
  bool ok = false;
  int M = 0, dsub = 0, D = 0, KC = 0, xexp = 0;
  int nref = 0;  // roundings of one term in the reference's distance (the bound's gamma)
  uint32_t nlist = 0;
  uint64_t nblocks = 0, max_blocks = 0;
  float cmax = 0.0f;  // largest |codebook component|
  // d_codes [N][M] in list order, offsets [nlist+1] (host), d_off the same
  // offsets on the device
  void build(const float* d_codebooks, const uint8_t* d_codes, const uint32_t* d_off,
             const std::vector<uint64_t>& offsets, uint32_t nlist, int M, int dsub, hipStream_t s);
  // The same blocks over full vectors: d_rows [N][dim] in list order (the
  // IVF index's lists); x^ is the row itself (M = 1, dsub = dim).
  void build_rows(const float* d_rows, const uint32_t* d_off, const std::vector<uint64_t>& offsets, uint32_t nlist,
                  int dim, hipStream_t s);
  DevBuf<uint4> data;
  DevBuf<float> xnb, cb4;  // cb4: codewords padded to a multiple of 4 floats
  DevBuf<uint32_t> xmax2, bo, stats;
};

// One screened batch, with the inputs the table scan takes.
struct Pq16SearchArgs {
  const float* queries;
  uint64_t nq;
  const int32_t* probes;  // [nq][np]
  int np;
  const float* centroids;
  const float* codebooks;
  const uint8_t* codes;
  const uint64_t* ids;
  const uint32_t* list_off;  // [nlist+1]
  int k;
  int order;  // AdcOrder of the exact distances
  // Full vectors (lists built with build_rows): rows [N][dim] in list order;
  // the query is the residual (centroids unused) and the exact distance is
  // the reference's squared L2, or its square root with sqrt_out (the
  // Euclidean metric); codebooks and codes are unused.
  const float* rows = nullptr;
  int sqrt_out = 0;
  // Work schedule: -1 by index size (tiles sorted by size and taken from
  // per-XCD counters when the index has at least 512 blocks per CU), 0 a
  // static stride over tiles in list order, 1 sorted tiles from counters.
  int tiles = -1;
  uint64_t* out_ids;
  float* out_d;
  uint32_t* out_counts;
};

class Pq16Searcher {
 public:
  Pq16Searcher() = default;
  Pq16Searcher(const Pq16Searcher&) = delete;
  Pq16Searcher& operator=(const Pq16Searcher&) = delete;
  ~Pq16Searcher();
  // Candidate entries per query (a query with more is rescanned exactly).
  // An entry is one lane's passing rows of one block: a row base, the probe
  // index and a 16-row mask.
  static uint32_t capacity(int k) { return k <= 64 ? 2048u : 16384u; }
  // Screened values kept per query from its first lists for the d_k bound
  // (a multiple of 32): more give a tighter bound and fewer candidates.
  // Measured at 1M x 128, k 10: 640 values gave 49 candidates per query and
  // the fastest step (1,024: 39, 2,048: 32, both slower overall).
  static uint32_t cap_first(int k) { return (uint32_t)std::min(4096, std::max(512, 64 * k)); }
  // Queries per slice, so the candidate buffer stays within 2 GiB.
  static uint64_t slice(int k) { return (1ull << 28) / capacity(k); }
  // Screens and rescores one slice (nq <= slice(k)); flags [nq] comes back
  // 1 for the queries left to the exact scan, 0 for those written.
  void search(const Pq16Lists& L, const Pq16SearchArgs& a, hipStream_t s);
  const int* flags() const { return flags_.p; }
  // Queries rescanned and candidates rescored since reset_stats, counted
  // when read (or when the next slice is searched).
  void reset_stats(hipStream_t s);
  void read_stats(uint64_t& fallbacks, uint64_t& candidates, hipStream_t s);
  // With timing on, search() brackets the threshold screening kernel with
  // events, waits for it and adds its duration to screen_ms() (cleared by
  // set_timing).
  void set_timing(bool on);
  float screen_ms() const { return screen_ms_; }

 private:
  void flush_stats(hipStream_t s);
  int ncu_ = 0;
  std::vector<std::pair<const void*, unsigned>> grids_;  // screening kernel -> its resident grid
  bool clear_ = true;        // the next count replaces stat_
  uint64_t pending_nq_ = 0;  // queries of the last slice, not yet counted
  bool timing_ = false;
  float screen_ms_ = 0.0f;
  hipEvent_t tev_[2] = {nullptr, nullptr};
  bool cnt_clean_ = false;  // cnt_ holds zeros
  DevBuf<uint32_t> cnt_, qoff_, toff_, tcnt_, tctr_, jlim_, offA_, nA_, nreal_, ccnt_, stat_, nheavy_, order_;
  DevBuf<uint2> qlist_, cand_, heavy_, multi_;
  DevBuf<uint4> desc_;  // tile descriptors of both stages
  DevBuf<uint32_t> part_k_;
  DevBuf<float> epsA_, bufA_, dkA_, part_d_;
  DevBuf<int> force_, flags_;
};

}  // namespace fdb
