// Host-side launchers for the forge-db HIP kernels.  All pointers are device
// pointers; every launcher enqueues on `stream` and returns the launch status.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fdb {

// Exact squared-L2 coarse selection.  For each of nq queries ([nq][dim]) the
// nsel nearest of nlist centroids, ascending by (distance, index), where the
// distance is computed in the reference's AVX2 order.  centT is the centroid
// matrix transposed to [dim][nlist] with dimensions permuted so that the 8
// FMA lanes read contiguous rows (see permute_dim).  nsel <= 1024.
// err_flag (nullable) is OR-ed with 1 when a distance is NaN.
// With a workspace part_d / part_k of part_cap entries (>= nq *
// coarse_parts(nq, nlist, nsel) * nsel), a batch too small to fill the GPU
// splits the centroids into coarse_parts(...) parts, each selecting its own
// list, and a second kernel merges them; the result is the same.  With
// only (nullable, [nq]), just the workgroups holding a query whose flag is
// set run (one part).
hipError_t launch_coarse_select(const float* queries, uint64_t nq, int dim, const float* centT,
                                int nlist, int nsel, int32_t* out_lists, float* out_dists,
                                int* err_flag, hipStream_t stream, float* part_d = nullptr,
                                uint32_t* part_k = nullptr, uint64_t part_cap = 0,
                                const int* only = nullptr);
// Number of centroid parts launch_coarse_select uses for this batch (1 = none).
int coarse_parts(uint64_t nq, int nlist, int nsel);

// Leading dimension of centT: rows are padded to a multiple of 256 columns
// (the coarse kernel reads 256 centroids per sweep); padding is zero.
__host__ __device__ inline int centT_ld(int k) { return (k + 255) / 256 * 256; }

// Row of the permuted dimension order used by centT: for the 8*floor(dim/8)
// leading dimensions, dim 8*i + l sits at row l*floor(dim/8) + i; the tail
// dimensions keep their place.
inline int permute_dim(int d, int dim) {
  const int d8 = dim / 8;
  if (d >= 8 * d8) return d;
  return (d % 8) * d8 + d / 8;
}

// Fused IVF-PQ scan: per query, residual LUTs for its probed lists built in
// LDS in the reference order, ADC over every code of those lists, wave64
// top-k, and a final merge.  Writes ids/dists [nq][k] ascending and
// counts [nq].  order: 0 = batch_search's 8-lane sum, 1 = search()'s groups
// of four.  probes: [nq][np] list ids.
struct IvfPqScanArgs {
  const float* queries;
  uint64_t nq;
  int dim, M, dsub;
  const int32_t* probes;  // entries outside [0, nlist) are skipped
  int np;
  int pstride;  // probes of query q start at q * pstride (0: np); the first np are scanned
  int nlist;
  const float* centroids;  // [nlist][dim]
  const float* codebooks;  // [M][256][dsub]
  const uint32_t* list_off;  // [nlist+1]
  const uint8_t* codes;      // [N][M], list order
  const uint64_t* ids;       // [N], list order
  int k;
  int order;
  // LUT mode: 0 = exact (the reference's rounding, bit-exact distances);
  // 1 = fast: T[m][j] = |cb_mj|^2 - 2<r_m, cb_mj> by FMA, with |r|^2 added
  // once per code (same quantity, different rounding).  Fast mode needs
  // cbnorm [M][256] = |cb_mj|^2 and the (16,8) or (32,3) shape.
  int lut_mode;
  const float* cbnorm;
  uint64_t* out_ids;
  float* out_dists;
  uint32_t* out_pos;  // nullable: list positions of the results
  uint32_t* out_counts;
  const uint32_t* live;  // nullable: bitmap over list positions, clear bit = skip
  const int* flags;      // nullable: [nq]; queries with a zero flag are not scanned
};
hipError_t launch_ivfpq_scan(const IvfPqScanArgs& a, hipStream_t stream);

// Bitmap over n list positions: bit p = (live == nullptr or live bit p) and
// ids[p] is in allowed (sorted ascending, n_allowed entries).
hipError_t launch_filter_bitmap(const uint64_t* ids, uint64_t n, const uint64_t* allowed,
                                uint64_t n_allowed, const uint32_t* live, uint32_t* out,
                                hipStream_t stream);

// |cb_mj|^2 for every codeword: [M*256]
hipError_t launch_codebook_norms(const float* codebooks, int M, int dsub, float* out,
                                 hipStream_t stream);

// Nearest row (first minimum) for each of n points, reference order; used for
// k-means assignment and list assignment at build time.  Same layout rules
// as launch_coarse_select.
inline hipError_t launch_assign(const float* points, uint64_t n, int dim, const float* centT,
                                int k, int32_t* out, hipStream_t stream) {
  return launch_coarse_select(points, n, dim, centT, k, 1, out, nullptr, nullptr, stream);
}

// k-means centroid update: for each cluster the f32 mean of its members
// summed in point order (src/kmeans.rs:165-185); clusters without members
// keep their previous row.  members: point indices grouped by cluster in
// ascending point order, member_off: [k+1].
hipError_t launch_kmeans_update(const float* points, int dim, const uint32_t* members,
                                const uint32_t* member_off, int k, const float* old_cents,
                                float* new_cents, hipStream_t stream);

// PQ encode of residuals x - centroid[list] for points in list order
// (src/pq.rs:114-139 applied as in src/index/ivf_pq.rs:450-478).
// rows: [n] point indices into vectors; row_list: [n] list of each row.
hipError_t launch_pq_encode(const float* vectors, const uint64_t* rows, const int32_t* row_list,
                            uint64_t n, int dim, const float* centroids, const float* codebooks,
                            int M, int dsub, uint8_t* codes, hipStream_t stream);

// Transpose + permute centroids [k][dim] into centT [dim][centT_ld(k)].
hipError_t launch_transpose_centroids(const float* cents, int k, int dim, float* centT,
                                      hipStream_t stream);

}  // namespace fdb
