// extern "C" boundary: the functions declared in include/forgedb_hip.h.
// Every entry point catches C++ exceptions and turns them into an
// fdb_status plus a thread-local message.
#include <cmath>
#include <cstring>
#include <string>

#include "fdb_flat.hpp"
#include "fdb_format.hpp"
#include "fdb_host.hpp"
#include "fdb_ivfpq.hpp"
#include "forgedb_hip.h"

struct fdb_ivfpq {
  fdb::IvfPqIndex* impl;
};
struct fdb_bf {
  fdb::BruteForceIndex* impl;
};
struct fdb_ivf {
  fdb::IvfFlatIndex* impl;
};

namespace fdb {

namespace {
thread_local std::string g_last_error;
}

void set_last_error(const std::string& msg) { g_last_error = msg; }

template <class F>
fdb_status guarded(F&& f) {
  try {
    f();
    return FDB_OK;
  } catch (const Error& e) {
    set_last_error(e.what());
    return e.status;
  } catch (const std::bad_alloc&) {
    set_last_error("host allocation failed");
    return FDB_ERR_OUT_OF_MEMORY;
  } catch (const std::exception& e) {
    set_last_error(e.what());
    return FDB_ERR_HIP;
  }
}

void require_device() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    throw Error(FDB_ERR_NO_DEVICE, "no HIP device visible");
  }
}

// Checks that flat artifacts describe a consistent index.
void validate(const IvfPqArtifacts& a) {
  if (a.nlist == 0 || a.dim == 0 || a.M == 0 || a.dim % a.M != 0)
    throw Error(FDB_ERR_INVALID_ARGUMENT, "nlist, dim and M must be positive with M dividing dim");
  if (a.metric > 4) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown metric");
  if (a.offsets.size() != (size_t)a.nlist + 1 || a.offsets[0] != 0)
    throw Error(FDB_ERR_INVALID_ARGUMENT, "list_offsets must have nlist+1 entries starting at 0");
  for (uint32_t l = 0; l < a.nlist; ++l)
    if (a.offsets[l + 1] < a.offsets[l]) throw Error(FDB_ERR_INVALID_ARGUMENT, "list_offsets decrease");
  if (a.dim > 2048) throw Error(FDB_ERR_UNSUPPORTED, "dim above 2048");
  if (a.M > 128) throw Error(FDB_ERR_UNSUPPORTED, "more than 128 subvectors");
}

fdb::IvfPqIndex* H(fdb_ivfpq* h) {
  if (!h || !h->impl) throw Error(FDB_ERR_INVALID_ARGUMENT, "null index handle");
  return h->impl;
}
const fdb::IvfPqIndex* H(const fdb_ivfpq* h) {
  if (!h || !h->impl) throw Error(FDB_ERR_INVALID_ARGUMENT, "null index handle");
  return h->impl;
}

template <class Handle>
auto* impl_of(Handle* h) {
  if (!h || !h->impl) throw Error(FDB_ERR_INVALID_ARGUMENT, "null index handle");
  return h->impl;
}

fdb_ivfpq* wrap(IvfPqArtifacts&& a) {
  validate(a);
  auto* impl = new fdb::IvfPqIndex(std::move(a));
  return new fdb_ivfpq{impl};
}

}  // namespace fdb

using namespace fdb;

extern "C" {

const char* fdb_last_error(void) { return g_last_error.c_str(); }
const char* fdb_version(void) { return "forgedb-hip 0.1 gfx950"; }

fdb_status fdb_ivfpq_create(const float* centroids, uint32_t nlist, uint32_t dim,
                            const float* codebooks, uint32_t M, const uint64_t* list_offsets,
                            const uint64_t* ids, const uint8_t* codes, uint32_t metric,
                            fdb_ivfpq** out) {
  return guarded([&] {
    if (!out || !centroids || !codebooks || !list_offsets)
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (nlist == 0 || dim == 0 || M == 0 || dim % M != 0)
      throw Error(FDB_ERR_INVALID_ARGUMENT, "nlist, dim and M must be positive with M dividing dim");
    require_device();
    IvfPqArtifacts a;
    a.nlist = nlist;
    a.dim = dim;
    a.M = M;
    a.dsub = dim / M;
    a.metric = metric;
    a.centroids.assign(centroids, centroids + (size_t)nlist * dim);
    a.codebooks.assign(codebooks, codebooks + (size_t)M * 256 * a.dsub);
    a.offsets.assign(list_offsets, list_offsets + nlist + 1);
    const uint64_t n = a.offsets.back();
    if (n && (!ids || !codes)) throw Error(FDB_ERR_INVALID_ARGUMENT, "null ids or codes");
    if (n) {
      a.ids.assign(ids, ids + n);
      a.codes.assign(codes, codes + n * M);
    }
    *out = wrap(std::move(a));
  });
}

fdb_status fdb_ivfpq_build(const float* vectors, const uint64_t* ids, uint64_t n, uint32_t dim,
                           uint32_t n_clusters, uint32_t M, uint32_t metric, uint64_t seed,
                           fdb_ivfpq** out) {
  return guarded([&] {
    if (!out || !vectors) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    require_device();
    IvfPqArtifacts a = IvfPqIndex::build(vectors, ids, n, dim, n_clusters, M, metric, seed);
    *out = wrap(std::move(a));
  });
}

fdb_status fdb_ivfpq_load(const char* path, fdb_ivfpq** out) {
  return guarded([&] {
    if (!out || !path) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    MappedFile file;
    IoResult r = map_file(path, file);
    if (r.status) throw Error(r.status, r.message);
    size_t off = 0;
    r = verify_header(file.data(), file.size(), IndexType::IvfPq, off);
    if (r.status) throw Error(r.status, r.message);
    IvfPqArtifacts a;
    r = decode_ivfpq(file.data() + off, file.size() - off, a);
    if (r.status) throw Error(r.status, r.message);
    require_device();
    *out = wrap(std::move(a));
  });
}

fdb_status fdb_ivfpq_save(const fdb_ivfpq* h, const char* path) {
  return guarded([&] {
    if (!path) throw Error(FDB_ERR_INVALID_ARGUMENT, "null path");
    const IvfPqIndex* ix = H(h);
    IvfPqArtifacts a = ix->artifacts();  // copy: nprobe reflects the live value
    a.nprobe = ix->nprobe();
    IoResult r = write_file(path, IndexType::IvfPq, encode_ivfpq(a));
    if (r.status) throw Error(r.status, r.message);
  });
}

void fdb_ivfpq_destroy(fdb_ivfpq* h) {
  if (!h) return;
  delete h->impl;
  delete h;
}

void fdb_ivfpq_set_nprobe(fdb_ivfpq* h, uint64_t nprobe) {
  if (h && h->impl) h->impl->set_nprobe(nprobe);
}

uint64_t fdb_ivfpq_nprobe(const fdb_ivfpq* h) { return (h && h->impl) ? h->impl->nprobe() : 0; }

fdb_status fdb_ivfpq_set_lut_mode(fdb_ivfpq* h, uint32_t mode) {
  return guarded([&] {
    if (mode > 1) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown LUT mode");
    if (!H(h)->set_lut_mode((int)mode))
      throw Error(FDB_ERR_UNSUPPORTED, "fast LUTs need 16 x 8 or 32 x 3 subvectors");
  });
}

uint32_t fdb_ivfpq_lut_mode(const fdb_ivfpq* h) {
  return (h && h->impl) ? (uint32_t)h->impl->lut_mode() : 0;
}

fdb_status fdb_ivfpq_set_coarse_mode(fdb_ivfpq* h, uint32_t mode) {
  return guarded([&] {
    if (mode > 2) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown coarse mode");
    H(h)->set_coarse_mode((int)mode);
  });
}

fdb_status fdb_ivfpq_set_search_mode(fdb_ivfpq* h, uint32_t mode) {
  return guarded([&] {
    if (!H(h)->set_search_mode((int)mode)) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown search mode");
  });
}

fdb_status fdb_ivfpq_last_screen_stats(fdb_ivfpq* h, void* stream, uint64_t* fallbacks, uint64_t* candidates) {
  return guarded([&] {
    if (!fallbacks || !candidates) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    H(h)->last_screen_stats(*fallbacks, *candidates, (hipStream_t)stream);
  });
}

fdb_status fdb_ivfpq_last_search_path(fdb_ivfpq* h, uint32_t* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = (uint32_t)H(h)->last_search_path();
  });
}

fdb_status fdb_ivfpq_last_screen_kernel_ms(fdb_ivfpq* h, float* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = H(h)->last_screen_kernel_ms();
  });
}

fdb_status fdb_ivfpq_describe(const fdb_ivfpq* h, fdb_ivfpq_desc* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    const IvfPqArtifacts& a = H(h)->artifacts();
    out->nlist = a.nlist;
    out->dim = a.dim;
    out->n_subvectors = a.M;
    out->subvector_dim = a.dsub;
    out->n_vectors = a.ids.size();
    out->metric = a.metric;
    out->reranking = a.has_originals ? 1 : 0;
    out->rerank_factor = a.rerank_factor;
  });
}

fdb_status fdb_ivfpq_export(const fdb_ivfpq* h, float* centroids, float* codebooks,
                            uint64_t* list_offsets, uint64_t* ids, uint8_t* codes) {
  return guarded([&] {
    const IvfPqArtifacts& a = H(h)->artifacts();
    if (centroids) std::memcpy(centroids, a.centroids.data(), 4 * a.centroids.size());
    if (codebooks) std::memcpy(codebooks, a.codebooks.data(), 4 * a.codebooks.size());
    if (list_offsets) std::memcpy(list_offsets, a.offsets.data(), 8 * a.offsets.size());
    if (ids) std::memcpy(ids, a.ids.data(), 8 * a.ids.size());
    if (codes) std::memcpy(codes, a.codes.data(), a.codes.size());
  });
}

fdb_status fdb_ivfpq_enable_reranking(fdb_ivfpq* h, const float* v, uint64_t factor) {
  return guarded([&] {
    if (!v) throw Error(FDB_ERR_INVALID_ARGUMENT, "null vectors");
    H(h)->enable_reranking(v, factor);
  });
}

fdb_status fdb_ivfpq_search(fdb_ivfpq* h, const float* query, uint32_t dim, uint32_t k,
                            uint64_t* out_ids, float* out_dists, uint32_t* out_count) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    if (!query || !out_count || (k && (!out_ids || !out_dists)))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    *out_count = ix->search(query, k, out_ids, out_dists);
  });
}

fdb_status fdb_ivfpq_batch_search(fdb_ivfpq* h, const float* queries, uint64_t nq, uint32_t dim,
                                  uint32_t k, uint64_t* out_ids, float* out_dists,
                                  uint32_t* out_counts) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    if (nq && (!queries || !out_counts || (k && (!out_ids || !out_dists))))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    ix->batch_search(queries, nq, k, out_ids, out_dists, out_counts);
  });
}

fdb_status fdb_ivfpq_batch_search_device(fdb_ivfpq* h, const float* d_queries, uint64_t nq,
                                         uint32_t k, uint64_t* d_out_ids, float* d_out_dists,
                                         uint32_t* d_out_counts, void* stream) {
  return guarded([&] {
    H(h)->batch_search_device(d_queries, nq, k, d_out_ids, d_out_dists, d_out_counts,
                              (hipStream_t)stream);
  });
}

fdb_status fdb_ivfpq_batch_search_device_timed(fdb_ivfpq* h, const float* d_queries, uint64_t nq,
                                               uint32_t k, uint64_t* d_out_ids, float* d_out_dists,
                                               uint32_t* d_out_counts, void* stream,
                                               float* coarse_ms, float* scan_ms) {
  return guarded([&] {
    float c = 0.0f, s = 0.0f;
    H(h)->batch_search_device(d_queries, nq, k, d_out_ids, d_out_dists, d_out_counts,
                              (hipStream_t)stream, &c, &s);
    if (coarse_ms) *coarse_ms = c;
    if (scan_ms) *scan_ms = s;
  });
}

fdb_status fdb_ivfpq_batch_search_device_noalloc(fdb_ivfpq* h, const float* d_queries, uint64_t nq,
                                                 uint32_t k, uint64_t* d_out_ids, float* d_out_dists,
                                                 uint32_t* d_out_counts, void* stream) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    uint64_t cap = 0;
    int32_t* probes = noalloc_scratch(cap);
    ix->batch_search_device_noalloc(d_queries, nq, k, d_out_ids, d_out_dists, d_out_counts, (hipStream_t)stream,
                                    probes, cap);
  });
}

fdb_status fdb_ivfpq_sync(fdb_ivfpq* h, void* stream) {
  return guarded([&] {
    if (H(h)->sync((hipStream_t)stream)) throw Error(FDB_ERR_NAN, "NaN centroid distance (a query contains NaN)");
  });
}

fdb_status fdb_ivfpq_probe(fdb_ivfpq* h, const float* queries, uint64_t nq, uint32_t dim,
                           uint32_t nprobe, int32_t* out_lists, float* out_dists) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    if (nq && (!queries || !out_lists)) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    ix->probe(queries, nq, nprobe, out_lists, out_dists);
  });
}

fdb_status fdb_ivfpq_encode(fdb_ivfpq* h, const float* residuals, uint64_t nq, uint32_t dim,
                            uint8_t* out_codes) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    if (nq && (!residuals || !out_codes)) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "vector dimension does not match the index");
    ix->encode(residuals, nq, out_codes);
  });
}

fdb_status fdb_ivfpq_search_filtered(fdb_ivfpq* h, const float* queries, uint64_t nq, uint32_t dim,
                                     uint32_t k, const uint64_t* allowed, uint64_t n_allowed,
                                     uint64_t* out_ids, float* out_dists, uint32_t* out_counts) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    if (nq && (!queries || !out_counts || (k && (!out_ids || !out_dists))))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (n_allowed && !allowed) throw Error(FDB_ERR_INVALID_ARGUMENT, "null allowed ids");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    ix->search_filtered(queries, nq, k, allowed, n_allowed, out_ids, out_dists, out_counts);
  });
}

fdb_status fdb_ivfpq_delete(fdb_ivfpq* h, uint64_t id, int* deleted) {
  return guarded([&] {
    const bool r = H(h)->remove(id);
    if (deleted) *deleted = r ? 1 : 0;
  });
}

fdb_status fdb_ivfpq_insert(fdb_ivfpq* h, const float* vectors, const uint64_t* ids, uint64_t n,
                            uint32_t dim) {
  return guarded([&] {
    IvfPqIndex* ix = H(h);
    if (n && !vectors) throw Error(FDB_ERR_INVALID_ARGUMENT, "null vectors");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "vector dimension does not match the index");
    ix->insert(vectors, ids, n);
  });
}

fdb_status fdb_ivfpq_compact(fdb_ivfpq* h) {
  return guarded([&] { H(h)->compact(); });
}

uint64_t fdb_ivfpq_len(const fdb_ivfpq* h) { return (h && h->impl) ? h->impl->live_len() : 0; }
uint64_t fdb_ivfpq_num_tombstones(const fdb_ivfpq* h) {
  return (h && h->impl) ? h->impl->num_tombstones() : 0;
}

/* ---- brute force ---------------------------------------------------------- */

fdb_status fdb_bf_create(uint32_t metric, fdb_bf** out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (metric > 4) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown metric");
    require_device();
    auto* impl = new BruteForceIndex(metric);
    *out = new fdb_bf{impl};
  });
}

fdb_status fdb_bf_add(fdb_bf* h, const float* rows, const uint64_t* ids, uint64_t n, uint32_t dim) {
  return guarded([&] { impl_of(h)->add(rows, ids, n, dim); });
}

fdb_status fdb_bf_remove(fdb_bf* h, uint64_t id, int* removed) {
  return guarded([&] {
    const bool r = impl_of(h)->remove(id);
    if (removed) *removed = r ? 1 : 0;
  });
}

uint64_t fdb_bf_len(const fdb_bf* h) { return (h && h->impl) ? h->impl->size() : 0; }
uint32_t fdb_bf_dimension(const fdb_bf* h) { return (h && h->impl) ? h->impl->dim() : 0; }
uint32_t fdb_bf_metric(const fdb_bf* h) { return (h && h->impl) ? h->impl->metric() : 0; }

fdb_status fdb_bf_load(const char* path, fdb_bf** out) {
  return guarded([&] {
    if (!out || !path) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    MappedFile file;
    IoResult r = map_file(path, file);
    if (r.status) throw Error(r.status, r.message);
    size_t off = 0;
    r = verify_header(file.data(), file.size(), IndexType::BruteForce, off);
    if (r.status) throw Error(r.status, r.message);
    BruteForceArtifacts a;
    r = decode_bf(file.data() + off, file.size() - off, a);
    if (r.status) throw Error(r.status, r.message);
    if (a.dim > 0xFFFFFFFFull) throw Error(FDB_ERR_UNSUPPORTED, "dimension above 2^32");
    require_device();
    auto* impl = new BruteForceIndex(a.metric);
    try {
      if (a.n) impl->add(a.data.data(), a.ids.data(), a.n, (uint32_t)a.dim);
    } catch (...) {
      delete impl;
      throw;
    }
    *out = new fdb_bf{impl};
  });
}

fdb_status fdb_bf_save(const fdb_bf* h, const char* path) {
  return guarded([&] {
    if (!path) throw Error(FDB_ERR_INVALID_ARGUMENT, "null path");
    const BruteForceIndex* ix = impl_of(h);
    BruteForceArtifacts a;
    a.metric = ix->metric();
    a.n = ix->size();
    a.dim = ix->dim();
    a.ids = ix->ids();
    a.data = ix->rows();
    IoResult r = write_file(path, IndexType::BruteForce, encode_bf(a));
    if (r.status) throw Error(r.status, r.message);
  });
}

void fdb_bf_destroy(fdb_bf* h) {
  if (!h) return;
  delete h->impl;
  delete h;
}

fdb_status fdb_bf_export(const fdb_bf* h, float* rows, uint64_t* ids) {
  return guarded([&] {
    const BruteForceIndex* ix = impl_of(h);
    if (rows) std::memcpy(rows, ix->rows().data(), 4 * ix->rows().size());
    if (ids) std::memcpy(ids, ix->ids().data(), 8 * ix->ids().size());
  });
}

fdb_status fdb_bf_search(fdb_bf* h, const float* query, uint32_t dim, uint32_t k, uint64_t* out_ids,
                         float* out_dists, uint32_t* out_count) {
  return guarded([&] {
    BruteForceIndex* ix = impl_of(h);
    if (!query || !out_count || (k && (!out_ids || !out_dists)))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (ix->size() && dim != ix->dim())
      throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    if (!ix->size()) {
      *out_count = 0;
      return;
    }
    *out_count = ix->search(query, k, out_ids, out_dists);
  });
}

fdb_status fdb_bf_batch_search(fdb_bf* h, const float* queries, uint64_t nq, uint32_t dim, uint32_t k,
                               uint64_t* out_ids, float* out_dists, uint32_t* out_counts) {
  return guarded([&] {
    BruteForceIndex* ix = impl_of(h);
    if (nq && (!queries || !out_counts || (k && (!out_ids || !out_dists))))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (ix->size() && dim != ix->dim())
      throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    if (!ix->size()) {
      for (uint64_t q = 0; q < nq; ++q) {
        out_counts[q] = 0;
        for (uint32_t j = 0; j < k; ++j) {
          out_ids[q * k + j] = ~0ull;
          out_dists[q * k + j] = HUGE_VALF;
        }
      }
      return;
    }
    ix->batch_search(queries, nq, k, out_ids, out_dists, out_counts);
  });
}

fdb_status fdb_bf_batch_search_device(fdb_bf* h, const float* d_queries, uint64_t nq, uint32_t k,
                                      uint64_t* d_out_ids, float* d_out_dists, uint32_t* d_out_counts,
                                      void* stream, float* ms) {
  return guarded([&] {
    impl_of(h)->batch_search_device(d_queries, nq, k, d_out_ids, d_out_dists, d_out_counts,
                                    (hipStream_t)stream, ms);
  });
}

fdb_status fdb_bf_set_search_mode(fdb_bf* h, uint32_t mode) {
  return guarded([&] {
    if (mode > 3) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown search mode");
    impl_of(h)->set_screen_mode((int)mode);
  });
}

fdb_status fdb_bf_last_search_path(fdb_bf* h, uint32_t* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = (uint32_t)impl_of(h)->last_path();
  });
}

fdb_status fdb_bf_last_fallbacks(fdb_bf* h, void* stream, uint64_t* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = impl_of(h)->last_fallbacks((hipStream_t)stream);
  });
}

/* ---- IVF ------------------------------------------------------------------ */

fdb_status fdb_ivf_create(const float* centroids, uint32_t nlist, uint32_t dim,
                          const uint64_t* list_offsets, const uint64_t* ids, const float* rows,
                          uint32_t metric, fdb_ivf** out) {
  return guarded([&] {
    if (!out || !centroids || !list_offsets) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    require_device();
    auto* impl = new IvfFlatIndex(centroids, nlist, dim, list_offsets, ids, rows, metric);
    *out = new fdb_ivf{impl};
  });
}

fdb_status fdb_ivf_build(const float* vectors, const uint64_t* ids, uint64_t n, uint32_t dim,
                         uint32_t n_clusters, uint32_t metric, uint64_t seed, fdb_ivf** out) {
  return guarded([&] {
    if (!out || !vectors) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (metric > 4) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown metric");
    require_device();
    auto* impl = IvfFlatIndex::build(vectors, ids, n, dim, n_clusters, metric, 100, seed);
    *out = new fdb_ivf{impl};
  });
}

void fdb_ivf_destroy(fdb_ivf* h) {
  if (!h) return;
  delete h->impl;
  delete h;
}

void fdb_ivf_set_nprobe(fdb_ivf* h, uint64_t nprobe) {
  if (h && h->impl) h->impl->set_nprobe(nprobe);
}
fdb_status fdb_ivf_set_coarse_mode(fdb_ivf* h, uint32_t mode) {
  return guarded([&] {
    if (mode > 2) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown coarse mode");
    impl_of(h)->set_coarse_mode((int)mode);
  });
}
fdb_status fdb_ivf_set_search_mode(fdb_ivf* h, uint32_t mode) {
  return guarded([&] {
    if (mode > 2) throw Error(FDB_ERR_INVALID_ARGUMENT, "unknown search mode");
    impl_of(h)->set_search_mode((int)mode);
  });
}

fdb_status fdb_ivf_last_screen_kernel_ms(fdb_ivf* h, float* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = impl_of(h)->last_screen_kernel_ms();
  });
}

fdb_status fdb_ivf_last_fallbacks(fdb_ivf* h, void* stream, uint64_t* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = impl_of(h)->last_fallbacks((hipStream_t)stream);
  });
}

fdb_status fdb_ivf_last_search_path(fdb_ivf* h, uint32_t* out) {
  return guarded([&] {
    if (!out) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    *out = (uint32_t)impl_of(h)->last_path();
  });
}

uint64_t fdb_ivf_nprobe(const fdb_ivf* h) { return (h && h->impl) ? h->impl->nprobe() : 0; }
uint64_t fdb_ivf_len(const fdb_ivf* h) { return (h && h->impl) ? h->impl->size() : 0; }
uint32_t fdb_ivf_num_partitions(const fdb_ivf* h) { return (h && h->impl) ? h->impl->nlist() : 0; }
uint32_t fdb_ivf_dimension(const fdb_ivf* h) { return (h && h->impl) ? h->impl->dim() : 0; }

fdb_status fdb_ivf_export(const fdb_ivf* h, float* centroids, uint64_t* list_offsets, uint64_t* ids,
                          float* rows) {
  return guarded([&] { impl_of(h)->export_to(centroids, list_offsets, ids, rows); });
}

fdb_status fdb_ivf_search(fdb_ivf* h, const float* query, uint32_t dim, uint32_t k, uint64_t* out_ids,
                          float* out_dists, uint32_t* out_count) {
  return guarded([&] {
    IvfFlatIndex* ix = impl_of(h);
    if (!query || !out_count || (k && (!out_ids || !out_dists)))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    ix->batch_search(query, 1, k, out_ids, out_dists, out_count);
  });
}

fdb_status fdb_ivf_batch_search(fdb_ivf* h, const float* queries, uint64_t nq, uint32_t dim, uint32_t k,
                                uint64_t* out_ids, float* out_dists, uint32_t* out_counts) {
  return guarded([&] {
    IvfFlatIndex* ix = impl_of(h);
    if (nq && (!queries || !out_counts || (k && (!out_ids || !out_dists))))
      throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    ix->batch_search(queries, nq, k, out_ids, out_dists, out_counts);
  });
}

fdb_status fdb_ivf_batch_search_device(fdb_ivf* h, const float* d_queries, uint64_t nq, uint32_t k,
                                       uint64_t* d_out_ids, float* d_out_dists, uint32_t* d_out_counts,
                                       void* stream, float* coarse_ms, float* scan_ms) {
  return guarded([&] {
    impl_of(h)->batch_search_device(d_queries, nq, k, d_out_ids, d_out_dists, d_out_counts,
                                    (hipStream_t)stream, coarse_ms, scan_ms);
  });
}

fdb_status fdb_ivf_probe(fdb_ivf* h, const float* queries, uint64_t nq, uint32_t dim, uint32_t nprobe,
                         int32_t* out_lists) {
  return guarded([&] {
    IvfFlatIndex* ix = impl_of(h);
    if (nq && (!queries || !out_lists)) throw Error(FDB_ERR_INVALID_ARGUMENT, "null argument");
    if (dim != ix->dim()) throw Error(FDB_ERR_DIMENSION_MISMATCH, "query dimension does not match the index");
    ix->probe(queries, nq, nprobe, out_lists);
  });
}

fdb_status fdb_ivf_sync(fdb_ivf* h, void* stream) {
  return guarded([&] {
    if (impl_of(h)->sync((hipStream_t)stream))
      throw Error(FDB_ERR_NAN, "NaN centroid distance (a query contains NaN)");
  });
}

}  // extern "C"
