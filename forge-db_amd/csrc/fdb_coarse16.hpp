// Coarse selection (the nprobe nearest centroids per query, ascending by
// (squared L2, centroid index)) screened on the matrix cores, with exact
// rescoring of a short list in the reference's order; the result equals the
// exact kernel's (launch_coarse_select) bit for bit.
//
// Reference: find_nearest_partitions, src/index/ivf_pq.rs:538-553 (and the
// copies in batch_search, :865-888); IVFIndex's stable sort, src/index/
// ivf.rs:164-177.  Distances are euclidean_distance_squared
// (src/distance/simd.rs:335-366).
//
// Method.  Centroids and queries are scaled by powers of two so that their
// largest components lie in [2^12, 2^13), rounded to fp16, and multiplied
// on the matrix cores (v_mfma_f32_32x32x16_f16, fp32 accumulation).  The
// screened value s = |c|^2 - 2<q, c> (|c|^2 in fp32) plus |q|^2 is within
// eps(q) = c_dot |q| X' + c_sq (|q| + X')^2 of the reference's d (X' = the
// largest centroid norm plus a term for values in the fp16 subnormal range;
// see screen_eps_coeffs in fdb_host.hpp).  |q|^2 is common to a query's
// centroids, so it cancels from every comparison below.
//   A workgroup of 4 waves takes 32 queries; each wave screens a quarter of
//   the 32-centroid blocks, each lane 16 centroids of a block (half of it)
//   for its query.
//   Pass 1: each (wave, half-lane) keeps the m smallest minima of its
//   half-blocks.  They belong to distinct centroids, so with S the
//   nprobe-th smallest of all kept minima, nprobe centroids have s <= S:
//   the nprobe-th smallest d is at most S + |q|^2 + eps, and every centroid
//   of the top nprobe has s <= S + 2 eps = T.
//   Pass 2: the products again; every centroid with s <= T is a candidate.
//   Rescoring: the candidates' exact distances in the reference's order;
//   the candidate of rank r by (distance, centroid index) is probe r.
// A query is flagged (and its probes come from the exact kernel, run on
// the flagged queries only) when it holds NaN or a value fp16 cannot carry,
// or when its candidates exceed the short list.
#pragma once

#include <stdint.h>

#include "fdb_host.hpp"

namespace fdb {

class Coarse16 {
 public:
  // Builds the fp16 centroid blocks from device centroids [nlist][dim];
  // usable() is false when a centroid is not finite, a component's scale
  // is out of range, or the shape is not served (dim > 256).
  void build(const float* d_centroids, uint32_t nlist, uint32_t dim, hipStream_t s);
  bool usable() const { return ok_; }
  // whether a selection of np probes is served (else: the exact kernel)
  bool serves(uint32_t np) const { return ok_ && np >= 1 && np <= 64 && np < nlist_ && np <= nblk_; }
  // probes [nq][np] ascending by (distance, index); dists [nq][np]
  // (nullable); flags [nq] (1: the query needs the exact kernel); err gets 1
  // for a NaN query (the exact kernel reports it again).
  void select(const float* d_qs, uint64_t nq, uint32_t np, const float* d_centroids, int32_t* probes,
              float* dists, int* flags, hipStream_t s);

 private:
  bool ok_ = false;
  uint32_t nlist_ = 0, dim_ = 0;
  int KC_ = 0, xexp_ = 0;
  uint32_t nblk_ = 0;
  float c_dot_ = 0, c_sq_ = 0, cabs_ = 0, xnorm_ = 0;
  DevBuf<uint4> blocks_;  // [nblk][KC][64] A operands
  DevBuf<float> cnp_;     // [nblk][2][16]: each half-lane's 16 |c|^2 (+inf past nlist)
  DevBuf<uint32_t> stats_;
  DevBuf<uint32_t> cand_, ncand_;  // [nq][cap] screened candidates and their counts (per call)
};

}  // namespace fdb
