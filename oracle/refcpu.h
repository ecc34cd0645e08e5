/*
 * refcpu — CPU restatement of forge-db's query-side nearest-neighbour path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the oracle that the HIP path is
 * checked against, and the CPU baseline that bench.py times beside the GPU.
 * Nothing in the shipped library links, loads or calls it.
 *
 * It restates the reference's Rust CPU path with the same AVX2+FMA
 * instruction sequences, lane orders and summation orders, the same heap
 * rules and the same batch grouping and chunking, so that its floating-point
 * results are the ones the reference produces on the default (AVX2, no
 * AVX-512) x86-64 build:
 *   distances   src/distance/simd.rs:290-517, src/distance/scalar.rs:8-97,
 *               src/distance/mod.rs:40-48
 *   PQ          src/pq.rs:114-139 (encode), :149-189 (LUT), :193-245 and
 *               :266-485 (ADC orders)
 *   IVF-PQ      src/index/ivf_pq.rs:374-506 (build), :524-553 (nprobe and
 *               coarse), :556-677 (rerank + search), :850-1084 (batch)
 *   brute force src/index/brute_force.rs:105-225
 *   IVF-flat    src/index/ivf.rs:91-405
 *   k-means     src/kmeans.rs:87-193, :316-329 (trainer shape; seeded here)
 *
 * Deliberate differences, none of which changes a result beyond the
 * reference's own nondeterminism:
 *   - The reference's RNG is unseeded thread_rng; training here draws from
 *     a documented seeded generator (SplitMix64 stream), see fdbo_rng_*.
 *   - select_nth_unstable / BinaryHeap / HashMap iteration leave exact ties
 *     unspecified in the reference; here they resolve deterministically
 *     (coarse: lower centroid index first; lists visited in ascending id).
 *   - batch_asymmetric_distance_avx2 allocates a Vec per code (pq.rs:321);
 *     here the 4-query batch writes into a stack buffer (same arithmetic).
 */
#ifndef FORGEDB_REFCPU_H
#define FORGEDB_REFCPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* DistanceMetric ordinals, src/distance/mod.rs:17-32 and the brute-force
 * payload metric byte, src/index/brute_force.rs:282-288. */
enum { FDBO_EUCLIDEAN = 0, FDBO_EUCLIDEAN_SQ = 1, FDBO_COSINE = 2,
       FDBO_DOT = 3, FDBO_MANHATTAN = 4 };

/* ---- distances: AVX2 dispatch path (what the default build runs) ---- */
float fdbo_l2sq(const float* a, const float* b, size_t n);   /* simd.rs:335-366 */
float fdbo_l2(const float* a, const float* b, size_t n);     /* simd.rs:290-328 */
float fdbo_dot(const float* a, const float* b, size_t n);    /* simd.rs:424-456 */
float fdbo_cosine(const float* a, const float* b, size_t n); /* simd.rs:466-517 */
float fdbo_l1(const float* a, const float* b, size_t n);     /* simd.rs:375-417 */
float fdbo_metric(int metric, const float* a, const float* b, size_t n); /* mod.rs:40-48 */
/* scalar twins, src/distance/scalar.rs:8-97 */
float fdbo_scalar_l2sq(const float* a, const float* b, size_t n);
float fdbo_scalar_dot(const float* a, const float* b, size_t n);
float fdbo_scalar_cosine(const float* a, const float* b, size_t n);
float fdbo_scalar_l1(const float* a, const float* b, size_t n);

/* ---- product quantizer ---- */
/* codebooks laid out [M][256][dsub] */
void fdbo_pq_lut(const float* codebooks, int M, int dsub, const float* r,
                 float* lut /* [M*256] */);                        /* pq.rs:175-189 */
float fdbo_adc_lanes8(const float* lut, const uint8_t* code, int M); /* pq.rs:435-485 */
float fdbo_adc_groups4(const float* lut, const uint8_t* code, int M);/* pq.rs:218-245 */
float fdbo_adc_seq(const float* lut, const uint8_t* code, int M);   /* pq.rs:410-418 */
void fdbo_adc_batch4(const float* const* luts, const uint8_t* code, int M,
                     float* out4);                                  /* pq.rs:318-402 */
void fdbo_pq_encode(const float* codebooks, int M, int dsub, const float* x,
                    uint8_t* code);                                 /* pq.rs:114-139 */

/* ---- seeded generator shared with the data generator ---- */
uint64_t fdbo_splitmix64_at(uint64_t seed, uint64_t i);
void fdbo_shuffle_indices(uint64_t seed, uint64_t* idx, uint64_t n);

/* ---- k-means (kmeans.rs:87-193), seeded ---- */
int fdbo_kmeans_fit(const float* data, uint64_t n, int dim, int k, int max_iters,
                    uint64_t seed, float* centroids_out /* [k*dim] */);

/* ---- IVF-PQ ---- */
typedef struct fdbo_ivfpq fdbo_ivfpq;
fdbo_ivfpq* fdbo_ivfpq_create(const float* centroids, int nlist, int dim,
                              const float* codebooks, int M,
                              const uint64_t* list_offsets /* [nlist+1] */,
                              const uint64_t* ids, const uint8_t* codes);
/* ivf_pq.rs:374-506 with seeded sampling; returns NULL on bad arguments */
fdbo_ivfpq* fdbo_ivfpq_build(const float* vectors, uint64_t n, int dim, int nlist,
                             int M, uint64_t seed, int nthreads);
void fdbo_ivfpq_destroy(fdbo_ivfpq* h);
void fdbo_ivfpq_shape(const fdbo_ivfpq* h, int* nlist, int* dim, int* M, uint64_t* n);
void fdbo_ivfpq_export(const fdbo_ivfpq* h, float* centroids, float* codebooks,
                       uint64_t* list_offsets, uint64_t* ids, uint8_t* codes);
void fdbo_ivfpq_set_nprobe(fdbo_ivfpq* h, uint64_t nprobe);          /* :524-527 */
uint64_t fdbo_ivfpq_nprobe(const fdbo_ivfpq* h);
/* rerank: original vectors in list order (same positions as codes), kept
   as a map id -> vector like original_vectors */
void fdbo_ivfpq_enable_reranking(fdbo_ivfpq* h, const float* vectors_list_order,
                                 uint64_t rerank_factor);            /* :513-517 */
/* original_vectors from (id, vector) records, rerank factor as stored */
void fdbo_ivfpq_set_originals(fdbo_ivfpq* h, const uint64_t* ids, const float* vectors,
                              uint64_t n, uint64_t rerank_factor);   /* :1918-1940 */
/* coarse selection as search() does it (:538-553); out sorted by (dist, idx) */
int fdbo_ivfpq_probes(const fdbo_ivfpq* h, const float* q, uint64_t nprobe,
                      int32_t* out_lists, float* out_dists);
/* search (:590-677): returns count, results ascending */
int fdbo_ivfpq_search(const fdbo_ivfpq* h, const float* q, int k,
                      uint64_t* out_ids, float* out_dists);
/* batch_search (:850-1047) over nq queries; out [nq][k], counts [nq] */
void fdbo_ivfpq_batch_search(const fdbo_ivfpq* h, const float* queries, uint64_t nq,
                             int k, uint64_t* out_ids, float* out_dists,
                             int32_t* out_counts);
/* search_filtered (:692-831), the filter as admitted ids; returns count */
int fdbo_ivfpq_search_filtered(const fdbo_ivfpq* h, const float* q, int k, const uint64_t* allowed,
                               uint64_t n_allowed, uint64_t* out_ids, float* out_dists);
/* delete (:1786-1804), insert_batch (:1731-1776), compact (:1828-1851) */
int fdbo_ivfpq_delete(fdbo_ivfpq* h, uint64_t id);
uint64_t fdbo_ivfpq_num_tombstones(const fdbo_ivfpq* h);
void fdbo_ivfpq_insert(fdbo_ivfpq* h, const float* vectors, const uint64_t* ids, uint64_t n);
void fdbo_ivfpq_compact(fdbo_ivfpq* h);
/* batch_search_parallel (:1060-1084) on nthreads (0 = all cores) */
void fdbo_ivfpq_batch_search_parallel(const fdbo_ivfpq* h, const float* queries,
                                      uint64_t nq, int k, int nthreads,
                                      uint64_t* out_ids, float* out_dists,
                                      int32_t* out_counts);

/* ---- brute force (brute_force.rs:105-225) ---- */
/* search over rows [N][dim] with ids; returns count */
int fdbo_bf_search(const float* data, const uint64_t* ids, uint64_t n, int dim,
                   int metric, const float* q, int k, uint64_t* out_ids, float* out_dists);
int fdbo_bf_search_parallel(const float* data, const uint64_t* ids, uint64_t n, int dim,
                            int metric, const float* q, int k, uint64_t* out_ids,
                            float* out_dists);
void fdbo_bf_batch_search(const float* data, const uint64_t* ids, uint64_t n, int dim,
                          int metric, const float* queries, uint64_t nq, int k,
                          int nthreads, uint64_t* out_ids, float* out_dists,
                          int32_t* out_counts);

/* ---- IVF-flat (ivf.rs:91-405); lists are CSR over list-ordered rows ---- */
int fdbo_ivf_probes(const float* centroids, int nlist, int dim, const float* q,
                    uint64_t nprobe, int32_t* out_lists);          /* ivf.rs:164-177 */
int fdbo_ivf_search(const float* centroids, int nlist, int dim,
                    const uint64_t* list_offsets, const uint64_t* ids,
                    const float* rows, int metric, uint64_t nprobe,
                    const float* q, int k, uint64_t* out_ids, float* out_dists);
void fdbo_ivf_batch_search(const float* centroids, int nlist, int dim,
                           const uint64_t* list_offsets, const uint64_t* ids,
                           const float* rows, int metric, uint64_t nprobe,
                           const float* queries, uint64_t nq, int k, int nthreads,
                           uint64_t* out_ids, float* out_dists, int32_t* out_counts);
/* ivf.rs:91-119 with a seeded k-means: centroids [nlist][dim], offsets
 * [nlist+1], order [n] = input row of each list-order position; 0 = ok */
int fdbo_ivf_build(const float* vectors, uint64_t n, int dim, int nlist, uint64_t seed,
                   int nthreads, float* centroids_out, uint64_t* offsets_out,
                   uint64_t* order_out);

#ifdef __cplusplus
}
#endif
#endif
