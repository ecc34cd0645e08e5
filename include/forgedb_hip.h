/*
 * forgedb_hip.h — C ABI of the MI355X (gfx950) query path for forge-db.
 *
 * Each entry point replaces one method of the reference's Rust API; the
 * reference file:line it stands in for is given beside it.  A Rust shim crate
 * binds these with `extern "C"` and keeps the reference's signatures
 * (infallible search methods panic with fdb_last_error() on a nonzero status).
 *
 * Conventions
 *   - Plain pointers and sizes only.  "host" buffers are ordinary CPU memory;
 *     "_device" entry points take device pointers and a hipStream_t (as void*,
 *     NULL = the handle's own stream) and only enqueue work.
 *   - Vectors and queries are row-major f32 [n][dim].
 *   - Result rows are [nq][k]: ids ascending by distance, then padding
 *     (id = UINT64_MAX, distance = +inf) after out_counts[q] valid entries.
 *   - Status: 0 = FDB_OK, negative = error; fdb_last_error() describes the
 *     last error on the calling thread.
 *   - Threading: a handle may be searched from several threads at once (calls
 *     on one handle serialise on its stream); set_nprobe may race with
 *     searches (relaxed atomic, as the reference's AtomicUsize).  Creating,
 *     loading and destroying need exclusive access.
 */
#ifndef FORGEDB_HIP_H
#define FORGEDB_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FDB_API __attribute__((visibility("default")))

typedef int32_t fdb_status;
enum {
  FDB_OK = 0,
  FDB_ERR_INVALID_ARGUMENT = -1,   /* ForgeDbError::InvalidParameter */
  FDB_ERR_DIMENSION_MISMATCH = -2, /* ForgeDbError::DimensionMismatch; the
                                      reference panics (pq.rs:150, simd.rs:339) */
  FDB_ERR_NAN = -3,                /* a NaN centroid distance; the reference
                                      panics in select_nth_unstable_by
                                      (ivf_pq.rs:547) */
  FDB_ERR_OUT_OF_MEMORY = -4,
  FDB_ERR_HIP = -5,                /* any other HIP runtime failure */
  FDB_ERR_IO = -6,                 /* ForgeDbError::Io */
  FDB_ERR_INVALID_FORMAT = -7,     /* ForgeDbError::InvalidFormat */
  FDB_ERR_CHECKSUM_MISMATCH = -8,  /* ForgeDbError::ChecksumMismatch */
  FDB_ERR_UNSUPPORTED = -9,        /* a size this build does not handle */
  FDB_ERR_NO_DEVICE = -10
};

/* DistanceMetric, src/distance/mod.rs:17-32 (same ordinals as the
 * brute-force payload metric byte, src/index/brute_force.rs:282-288). */
enum {
  FDB_METRIC_EUCLIDEAN = 0,
  FDB_METRIC_EUCLIDEAN_SQUARED = 1,
  FDB_METRIC_COSINE = 2,
  FDB_METRIC_DOT_PRODUCT = 3,
  FDB_METRIC_MANHATTAN = 4
};

FDB_API const char* fdb_last_error(void);
FDB_API const char* fdb_version(void);

/* ------------------------------------------------------------------------ */
/* IVF-PQ: src/index/ivf_pq.rs                                              */
/* ------------------------------------------------------------------------ */
typedef struct fdb_ivfpq fdb_ivfpq;

typedef struct {
  uint32_t nlist;        /* n_partitions(), ivf_pq.rs:1110 */
  uint32_t dim;          /* dim(), ivf_pq.rs:1121 */
  uint32_t n_subvectors; /* ProductQuantizer::n_subvectors, pq.rs:37 */
  uint32_t subvector_dim;
  uint64_t n_vectors;    /* len_with_tombstones(), ivf_pq.rs:1096 */
  uint32_t metric;
  uint32_t reranking;    /* 1 when original vectors are resident */
  uint64_t rerank_factor;
} fdb_ivfpq_desc;

/* Build from trained artifacts (the state IVFPQIndex::build leaves behind,
 * ivf_pq.rs:494-505).  centroids [nlist][dim]; codebooks [M][256][dim/M];
 * list_offsets [nlist+1] into ids [N] and codes [N][M], both in list order.
 * nprobe starts at 1 (ivf_pq.rs:501). */
FDB_API fdb_status fdb_ivfpq_create(const float* centroids, uint32_t nlist, uint32_t dim,
                                    const float* codebooks, uint32_t n_subvectors,
                                    const uint64_t* list_offsets, const uint64_t* ids,
                                    const uint8_t* codes, uint32_t metric, fdb_ivfpq** out);

/* IVFPQIndex::build, ivf_pq.rs:374-506, run on the GPU: k-means coarse
 * training on a 30k sample, list assignment, PQ training on a 100k residual
 * sample, residual encoding.  The reference draws its samples from an
 * unseeded thread_rng; here they come from the SplitMix64 streams
 * splitmix64(seed, 0|1|2|16+m).  ids may be NULL (ids 0..n-1). */
FDB_API fdb_status fdb_ivfpq_build(const float* vectors, const uint64_t* ids, uint64_t n,
                                   uint32_t dim, uint32_t n_clusters, uint32_t n_subvectors,
                                   uint32_t metric, uint64_t seed, fdb_ivfpq** out);

/* Persistable::load / load_mmap / save for IVF-PQ, ivf_pq.rs:1970-1994:
 * 24-byte header + CRC-32 (persistence/mod.rs:77-94,169-188) around the
 * bincode payload of SerializableIVFPQ (ivf_pq.rs:307-316). */
FDB_API fdb_status fdb_ivfpq_load(const char* path, fdb_ivfpq** out);
FDB_API fdb_status fdb_ivfpq_save(const fdb_ivfpq* index, const char* path);

FDB_API void fdb_ivfpq_destroy(fdb_ivfpq* index);

/* set_nprobe (ivf_pq.rs:524-527): stores min(nprobe, nlist), relaxed. */
FDB_API void fdb_ivfpq_set_nprobe(fdb_ivfpq* index, uint64_t nprobe);
/* nprobe() (ivf_pq.rs:1116-1118) */
FDB_API uint64_t fdb_ivfpq_nprobe(const fdb_ivfpq* index);

FDB_API fdb_status fdb_ivfpq_describe(const fdb_ivfpq* index, fdb_ivfpq_desc* out);

/* Lookup-table mode (no counterpart in the reference, whose CPU path has one
 * way of building tables):
 *   FDB_LUT_EXACT (default) builds T[m][j] = |r_m - cb_mj|^2 with the
 *     reference's operation order, so ADC distances are bit-identical;
 *   FDB_LUT_FAST builds |cb_mj|^2 - 2<r_m, cb_mj> by FMA and adds |r|^2 once
 *     per code: the same quantity within ~1e-6 relative, ~3x fewer table
 *     operations.  Available for 16 x 8 and 32 x 3 subvector shapes
 *     (FDB_ERR_UNSUPPORTED otherwise).  Relaxed atomic, like set_nprobe. */
enum { FDB_LUT_EXACT = 0, FDB_LUT_FAST = 1 };
FDB_API fdb_status fdb_ivfpq_set_lut_mode(fdb_ivfpq* index, uint32_t mode);
FDB_API uint32_t fdb_ivfpq_lut_mode(const fdb_ivfpq* index);

/* Coarse selection strategy (no counterpart in the reference):
 *   FDB_COARSE_AUTO (default) and FDB_COARSE_EXACT: the exact-order VALU
 *     kernel (faster at nlist <= 4096);
 *   FDB_COARSE_SCREEN: MFMA screening when nprobe + 16 <= 128 and dim is a
 *     multiple of 4 (<= 512).
 * Screening computes approximate distances on the matrix cores, recomputes
 * the best nprobe + 16..128 in the reference's order and proves from a
 * rounding-error bound that no other list belongs to the nprobe nearest;
 * queries where that fails go through the exact kernel.  The probed lists
 * and their distances are the same in every mode. */
enum { FDB_COARSE_AUTO = 0, FDB_COARSE_EXACT = 1, FDB_COARSE_SCREEN = 2 };
FDB_API fdb_status fdb_ivfpq_set_coarse_mode(fdb_ivfpq* index, uint32_t mode);

/* Scan strategy for batches (no counterpart in the reference, which scores
 * every code of the probed lists through the distance tables):
 *   FDB_IVFPQ_AUTO (default): batches scanning at least 2^26 codes with
 *     exact tables, no reranking, no tombstones and dim <= 256 are screened:
 *     the exact scan of each query's nearest probed list gives d_k (its k-th
 *     distance there); half-precision products of each residual with every
 *     decoded code of the other probed lists (matrix cores) select the codes
 *     whose screened distance is within a rounding-error bound of d_k; those
 *     are rescored exactly in the reference's order.  A code left out is
 *     provably farther than d_k, so results are identical to
 *     FDB_IVFPQ_EXACT.  Queries with more candidates than the buffer holds,
 *     or residuals out of half-precision range, are rescanned exactly.
 *   FDB_IVFPQ_EXACT: the table scan for every query.
 *   FDB_IVFPQ_SCREEN: screening wherever it applies, whatever the size.
 *   FDB_IVFPQ_SCREEN_SORTED: as FDB_IVFPQ_SCREEN, with the work schedule
 *     that large indexes take by themselves (tiles ordered by size, taken
 *     from per-XCD counters) whatever the index size; the same results.
 * fdb_ivfpq_last_screen_stats reports, for the last batch, the queries
 * rescanned exactly and the candidates rescored (waits for hip_stream; NULL
 * = the handle's stream); fdb_ivfpq_last_search_path 0 (table scan) or 2
 * (screening).  The decoded codes take 2 * roundup(dim, 16) bytes per code
 * of device memory, built at the first screened search after the lists
 * change. */
enum { FDB_IVFPQ_AUTO = 0, FDB_IVFPQ_EXACT = 1, FDB_IVFPQ_SCREEN = 2, FDB_IVFPQ_SCREEN_SORTED = 3 };
FDB_API fdb_status fdb_ivfpq_set_search_mode(fdb_ivfpq* index, uint32_t mode);
FDB_API fdb_status fdb_ivfpq_last_screen_stats(fdb_ivfpq* index, void* hip_stream, uint64_t* fallbacks,
                                               uint64_t* candidates);
FDB_API fdb_status fdb_ivfpq_last_search_path(fdb_ivfpq* index, uint32_t* out);
/* Measurement (no counterpart in the reference): the duration in ms of the
 * screening kernel that tests every probed code against its query's bound
 * (pq16_thresh_kernel, summed over slices) in the last call of
 * fdb_ivfpq_batch_search_device_timed, from HIP events on the call's
 * stream; 0 when that call took the table scan. */
FDB_API fdb_status fdb_ivfpq_last_screen_kernel_ms(fdb_ivfpq* index, float* out);

/* Copies the resident artifacts back (any pointer may be NULL). */
FDB_API fdb_status fdb_ivfpq_export(const fdb_ivfpq* index, float* centroids, float* codebooks,
                                    uint64_t* list_offsets, uint64_t* ids, uint8_t* codes);

/* enable_reranking (ivf_pq.rs:513-517): original vectors [N][dim] in list
 * order (the same positions as ids/codes); searches then fetch
 * k * rerank_factor ADC candidates and return exact sqrt(L2) re-ranked
 * results (rerank_results, ivf_pq.rs:556-582). */
FDB_API fdb_status fdb_ivfpq_enable_reranking(fdb_ivfpq* index, const float* vectors_list_order,
                                              uint64_t rerank_factor);

/* search (ivf_pq.rs:590-677): one query, its nprobe lists (0 lists when
 * nprobe is 0), ADC summed as asymmetric_distance_fast (pq.rs:218-245).
 * out_ids/out_dists hold k entries. */
FDB_API fdb_status fdb_ivfpq_search(fdb_ivfpq* index, const float* query, uint32_t dim,
                                    uint32_t k, uint64_t* out_ids, float* out_dists,
                                    uint32_t* out_count);

/* batch_search (ivf_pq.rs:850-1047) and batch_search_parallel (:1060-1084):
 * nq queries, max(nprobe,1) lists each, ADC summed in the 8-lane AVX2 order
 * (pq.rs:318-485).  Results [nq][k] in input order. */
FDB_API fdb_status fdb_ivfpq_batch_search(fdb_ivfpq* index, const float* queries, uint64_t nq,
                                          uint32_t dim, uint32_t k, uint64_t* out_ids,
                                          float* out_dists, uint32_t* out_counts);

/* The same with inputs and outputs already in device memory; enqueues only.
 * A NaN query is reported by the next fdb_ivfpq_sync. */
FDB_API fdb_status fdb_ivfpq_batch_search_device(fdb_ivfpq* index, const float* d_queries,
                                                 uint64_t nq, uint32_t k, uint64_t* d_out_ids,
                                                 float* d_out_dists, uint32_t* d_out_counts,
                                                 void* hip_stream);
/* No counterpart in the reference: fdb_ivfpq_batch_search_device for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  It allocates nothing:
 * the [nq][nprobe] probe lists go to a static device array of 2^21 int32
 * entries (8 MiB per device, held until the process ends), and the table
 * scan writes straight to the caller's outputs; the results equal
 * fdb_ivfpq_batch_search_device's.  FDB_ERR_UNSUPPORTED when nq * nprobe
 * exceeds 2^21, or the index has reranking on or tombstones.  Every call on
 * one device shares that array: calls that overlap on one device (other
 * handles or other streams included) race. */
FDB_API fdb_status fdb_ivfpq_batch_search_device_noalloc(fdb_ivfpq* index, const float* d_queries,
                                                         uint64_t nq, uint32_t k, uint64_t* d_out_ids,
                                                         float* d_out_dists, uint32_t* d_out_counts,
                                                         void* hip_stream);
/* Waits for the handle's work on `hip_stream` (NULL = own stream) and
 * returns FDB_ERR_NAN if a device search since the last sync saw a NaN. */
FDB_API fdb_status fdb_ivfpq_sync(fdb_ivfpq* index, void* hip_stream);

/* Coarse quantizer alone (find_nearest_partitions, ivf_pq.rs:538-553): the
 * nprobe nearest lists per query, ascending by (distance, list id), with the
 * exact reference-order squared distances. */
FDB_API fdb_status fdb_ivfpq_probe(fdb_ivfpq* index, const float* queries, uint64_t nq,
                                   uint32_t dim, uint32_t nprobe, int32_t* out_lists,
                                   float* out_dists);

/* ProductQuantizer::encode (pq.rs:114-139) of nq residual vectors [nq][dim]
 * against the index's codebooks: codes [nq][M]. */
FDB_API fdb_status fdb_ivfpq_encode(fdb_ivfpq* index, const float* residuals, uint64_t nq,
                                    uint32_t dim, uint8_t* out_codes);

/* search_filtered (ivf_pq.rs:692-831) for nq queries (nq = 1 is the
 * reference call): the metadata filter arrives already evaluated, as the
 * n_allowed vector ids it admits (MetadataStore::filter_bitmap mapped back to
 * ids, any order); only untombstoned entries with an admitted id are
 * scanned.  Like the reference: nprobe lists (0 when nprobe is 0), the
 * search() ADC order, 4 * k (* rerank_factor) candidates kept, then rerank
 * or truncation to k; no admitted id gives no results. */
FDB_API fdb_status fdb_ivfpq_search_filtered(fdb_ivfpq* index, const float* queries, uint64_t nq,
                                             uint32_t dim, uint32_t k, const uint64_t* allowed_ids,
                                             uint64_t n_allowed, uint64_t* out_ids,
                                             float* out_dists, uint32_t* out_counts);
/* delete (ivf_pq.rs:1786-1804): tombstones id in the first list that holds it
 * untombstoned; *deleted = 1 then, else 0.  Searches skip every entry of
 * that list with this id.  Tombstones are not saved (SerializablePartition
 * carries none, :222-243). */
FDB_API fdb_status fdb_ivfpq_delete(fdb_ivfpq* index, uint64_t id, int* deleted);
/* insert_batch (ivf_pq.rs:1731-1776): n vectors [n][dim] with ids (NULL:
 * len_with_tombstones()..+n-1) go to their nearest list (first minimum),
 * their residuals encoded with the codebooks, appended in input order; an
 * inserted id leaves that list's tombstones.  With reranking enabled the
 * vectors become the originals of the new entries. */
FDB_API fdb_status fdb_ivfpq_insert(fdb_ivfpq* index, const float* vectors, const uint64_t* ids,
                                    uint64_t n, uint32_t dim);
/* compact (ivf_pq.rs:1828-1851): removes tombstoned entries. */
FDB_API fdb_status fdb_ivfpq_compact(fdb_ivfpq* index);
/* len (:1088-1094, entries minus tombstones) and num_tombstones (:1807) */
FDB_API uint64_t fdb_ivfpq_len(const fdb_ivfpq* index);
FDB_API uint64_t fdb_ivfpq_num_tombstones(const fdb_ivfpq* index);

/* Kernel timing for measurement: runs one batch_search_device and returns the
 * durations in ms of the coarse and scan kernels (HIP events on the stream
 * they run on). */
FDB_API fdb_status fdb_ivfpq_batch_search_device_timed(fdb_ivfpq* index, const float* d_queries,
                                                       uint64_t nq, uint32_t k,
                                                       uint64_t* d_out_ids, float* d_out_dists,
                                                       uint32_t* d_out_counts, void* hip_stream,
                                                       float* coarse_ms, float* scan_ms);

/* ------------------------------------------------------------------------ */
/* Brute force: src/index/brute_force.rs                                    */
/* ------------------------------------------------------------------------ */
/* Distances are the metric's AVX2 form (src/distance/simd.rs:290-517, via
 * DistanceMetric::compute, distance/mod.rs:40-48), bit-identical.  Results
 * are the k smallest, ascending; equal distances keep the earlier row first
 * (the strict-< heap replacement of scan_range, brute_force.rs:141-146). */
typedef struct fdb_bf fdb_bf;

/* BruteForceIndex::new (brute_force.rs:67-72): empty; the first add fixes
 * the dimension. */
FDB_API fdb_status fdb_bf_create(uint32_t metric, fdb_bf** out);
/* add (brute_force.rs:75-80) for n rows [n][dim]; ids may be NULL (ids
 * len()..len()+n-1).  MutableVectorIndex::add (:254-265):
 * FDB_ERR_DIMENSION_MISMATCH when dim differs from a non-empty index. */
FDB_API fdb_status fdb_bf_add(fdb_bf* index, const float* rows, const uint64_t* ids, uint64_t n,
                              uint32_t dim);
/* MutableVectorIndex::remove (:267-274): *removed = 1 when a row had this
 * id; the last row takes its place (VectorStore::swap_remove). */
FDB_API fdb_status fdb_bf_remove(fdb_bf* index, uint64_t id, int* removed);
/* len (:83) and dimension (:95; 0 when empty) */
FDB_API uint64_t fdb_bf_len(const fdb_bf* index);
FDB_API uint32_t fdb_bf_dimension(const fdb_bf* index);
FDB_API uint32_t fdb_bf_metric(const fdb_bf* index);
/* Persistable for BruteForceIndex (:277-385): header + payload
 * [metric u8][n u64][dim u64][ids][data]. */
FDB_API fdb_status fdb_bf_load(const char* path, fdb_bf** out);
FDB_API fdb_status fdb_bf_save(const fdb_bf* index, const char* path);
FDB_API void fdb_bf_destroy(fdb_bf* index);
/* Copies rows [len][dim] and ids [len] out (either may be NULL). */
FDB_API fdb_status fdb_bf_export(const fdb_bf* index, float* rows, uint64_t* ids);
/* search / search_prefetch / search_parallel (:162-214): one query. */
FDB_API fdb_status fdb_bf_search(fdb_bf* index, const float* query, uint32_t dim, uint32_t k,
                                 uint64_t* out_ids, float* out_dists, uint32_t* out_count);
/* batch_search (:220-225): results [nq][k] in input order. */
FDB_API fdb_status fdb_bf_batch_search(fdb_bf* index, const float* queries, uint64_t nq,
                                       uint32_t dim, uint32_t k, uint64_t* out_ids,
                                       float* out_dists, uint32_t* out_counts);
/* Device-resident inputs/outputs; enqueues only.  ms (nullable): when given,
 * waits and returns the duration of the enqueued work (HIP events). */
FDB_API fdb_status fdb_bf_batch_search_device(fdb_bf* index, const float* d_queries, uint64_t nq,
                                              uint32_t k, uint64_t* d_out_ids, float* d_out_dists,
                                              uint32_t* d_out_counts, void* hip_stream, float* ms);

/* Search strategy (no counterpart in the reference, whose scan is one
 * loop):
 *   FDB_BF_AUTO (default) and FDB_BF_SCREEN: for dot product, cosine and
 *     (squared) Euclidean with dim a multiple of 4 (<= 512) and k <= 112,
 *     a matrix-core pass screens K' = 64 or 128 candidates per query, their
 *     distances are recomputed exactly in the reference's order, and a
 *     rounding-error bound proves that no other row can enter the top k;
 *     queries where it cannot be proved are rescanned exactly.  Results are
 *     identical to FDB_BF_EXACT.  The pass uses fp16 products when the rows
 *     fit (finite, no zero-norm rows for cosine), else fp32 products.
 *   FDB_BF_EXACT: the exact-order VALU scan for every query.
 *   FDB_BF_SCREEN_F32: screening with the fp32 products only.
 * fdb_bf_last_fallbacks reports how many queries of the last search were
 * rescanned (it waits for hip_stream; NULL = the handle's own stream). */
enum { FDB_BF_AUTO = 0, FDB_BF_EXACT = 1, FDB_BF_SCREEN = 2, FDB_BF_SCREEN_F32 = 3 };
FDB_API fdb_status fdb_bf_set_search_mode(fdb_bf* index, uint32_t mode);
FDB_API fdb_status fdb_bf_last_fallbacks(fdb_bf* index, void* hip_stream, uint64_t* out);
/* How the last search ran (diagnostics; no counterpart in the reference):
 * 0 exact scan, 1 fp32 screening, 2 fp16 screening. */
FDB_API fdb_status fdb_bf_last_search_path(fdb_bf* index, uint32_t* out);

/* ------------------------------------------------------------------------ */
/* IVF (full vectors): src/index/ivf.rs                                     */
/* ------------------------------------------------------------------------ */
/* Coarse: squared L2 to every centroid, stable ascending sort (ties → lower
 * list id), first nprobe lists (ivf.rs:164-177).  Scan: metric.compute over
 * every vector of those lists, bit-identical; the k smallest ascending, equal
 * distances ordered by list-order position. */
typedef struct fdb_ivf fdb_ivf;

/* From the state IVFIndex::build leaves (ivf.rs:113-118): centroids
 * [nlist][dim]; list_offsets [nlist+1] into ids [N] and rows [N][dim] in list
 * order.  nprobe starts at 1. */
FDB_API fdb_status fdb_ivf_create(const float* centroids, uint32_t nlist, uint32_t dim,
                                  const uint64_t* list_offsets, const uint64_t* ids,
                                  const float* rows, uint32_t metric, fdb_ivf** out);
/* IVFIndex::build (ivf.rs:91-119) on the GPU: k-means over all vectors with
 * DEFAULT_MAX_ITERATIONS = 100 (constants.rs:32), initialised from the
 * SplitMix64 stream splitmix64(seed, 1) (the reference draws from an unseeded
 * thread_rng), then first-minimum assignment; each list keeps input order.
 * ids may be NULL (0..n-1). */
FDB_API fdb_status fdb_ivf_build(const float* vectors, const uint64_t* ids, uint64_t n,
                                 uint32_t dim, uint32_t n_clusters, uint32_t metric, uint64_t seed,
                                 fdb_ivf** out);
FDB_API void fdb_ivf_destroy(fdb_ivf* index);
/* set_nprobe (ivf.rs:125-127): min(nprobe, nlist); nprobe() (:130-132) */
FDB_API void fdb_ivf_set_nprobe(fdb_ivf* index, uint64_t nprobe);
/* Coarse selection strategy, as fdb_ivfpq_set_coarse_mode. */
FDB_API fdb_status fdb_ivf_set_coarse_mode(fdb_ivf* index, uint32_t mode);
/* Scan strategy (no counterpart in the reference, whose scan is one loop):
 *   FDB_IVF_AUTO (default):
 *     - Euclidean and squared Euclidean batches of at least 2^26 (query,
 *       row) pairs (dim <= 256, nprobe >= 2): list screening.  The (query,
 *       list) pairs are grouped by list and each list's rows, in half
 *       precision, are multiplied against up to 256 queries at a time on the
 *       matrix cores; a rounding-error bound on the k-th distance keeps
 *       every row that can enter the top k, whose distances are then
 *       recomputed exactly in the reference's order.
 *     - else, for Euclidean, squared Euclidean and Manhattan with k <= 112
 *       and dim a multiple of 4 (<= 512): per-query screening.  The probed
 *       lists are scanned in half precision to pick K' = 64 or 128
 *       candidates per query, their distances are recomputed exactly, and a
 *       bound proves that no other scanned row can enter the top k.
 *     Queries where a bound cannot be proved are rescanned exactly.  Results
 *     are identical to FDB_IVF_EXACT.
 *   FDB_IVF_EXACT: the exact-order scan for every query.
 *   FDB_IVF_SCREEN_LISTS: list screening wherever it applies, whatever the
 *     batch size; otherwise as FDB_IVF_AUTO.
 * fdb_ivf_last_fallbacks counts the queries of the last search that were
 * rescanned (waits for hip_stream; NULL = the handle's own stream);
 * fdb_ivf_last_search_path reports 0 (exact scan), 2 (per-query screening)
 * or 3 (list screening). */
enum { FDB_IVF_AUTO = 0, FDB_IVF_EXACT = 1, FDB_IVF_SCREEN_LISTS = 2 };
/* Measurement (no counterpart in the reference): the duration in ms of the
 * list screening's threshold kernel (pq16_thresh_kernel, summed over
 * slices) in the last fdb_ivf_batch_search_device call given coarse_ms or
 * scan_ms, from HIP events on the call's stream; 0 when that call did not
 * take list screening. */
FDB_API fdb_status fdb_ivf_last_screen_kernel_ms(fdb_ivf* index, float* out);
FDB_API fdb_status fdb_ivf_set_search_mode(fdb_ivf* index, uint32_t mode);
FDB_API fdb_status fdb_ivf_last_fallbacks(fdb_ivf* index, void* hip_stream, uint64_t* out);
FDB_API fdb_status fdb_ivf_last_search_path(fdb_ivf* index, uint32_t* out);
FDB_API uint64_t fdb_ivf_nprobe(const fdb_ivf* index);
/* len (:135), num_partitions (:145), dimension (:150) */
FDB_API uint64_t fdb_ivf_len(const fdb_ivf* index);
FDB_API uint32_t fdb_ivf_num_partitions(const fdb_ivf* index);
FDB_API uint32_t fdb_ivf_dimension(const fdb_ivf* index);
/* Copies the artifacts back (any pointer may be NULL). */
FDB_API fdb_status fdb_ivf_export(const fdb_ivf* index, float* centroids, uint64_t* list_offsets,
                                  uint64_t* ids, float* rows);
/* search / search_parallel (ivf.rs:162-290): one query; nprobe 0 → empty. */
FDB_API fdb_status fdb_ivf_search(fdb_ivf* index, const float* query, uint32_t dim, uint32_t k,
                                  uint64_t* out_ids, float* out_dists, uint32_t* out_count);
/* batch_search / batch_search_optimized (ivf.rs:292-405): [nq][k]. */
FDB_API fdb_status fdb_ivf_batch_search(fdb_ivf* index, const float* queries, uint64_t nq,
                                        uint32_t dim, uint32_t k, uint64_t* out_ids,
                                        float* out_dists, uint32_t* out_counts);
/* Device-resident inputs/outputs; enqueues only (a NaN query is reported by
 * fdb_ivf_sync).  coarse_ms/scan_ms (nullable): when given, waits and returns
 * the two kernels' durations (HIP events). */
FDB_API fdb_status fdb_ivf_batch_search_device(fdb_ivf* index, const float* d_queries, uint64_t nq,
                                               uint32_t k, uint64_t* d_out_ids, float* d_out_dists,
                                               uint32_t* d_out_counts, void* hip_stream,
                                               float* coarse_ms, float* scan_ms);
FDB_API fdb_status fdb_ivf_sync(fdb_ivf* index, void* hip_stream);
/* Coarse step alone (ivf.rs:164-177): the nprobe (<= nlist) nearest lists
 * per query, ascending by (squared L2, list id). */
FDB_API fdb_status fdb_ivf_probe(fdb_ivf* index, const float* queries, uint64_t nq, uint32_t dim,
                                 uint32_t nprobe, int32_t* out_lists);

#ifdef __cplusplus
}
#endif
#endif
