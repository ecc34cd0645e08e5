// .fdb container and payload codecs.  See fdb_format.hpp for the layouts.
#include "fdb_format.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <unordered_map>

#include "forgedb_hip.h"

namespace fdb {

namespace {

const uint8_t kMagic[8] = {'F', 'O', 'R', 'G', 'E', 'D', 'B', 0};
constexpr uint32_t kFormatVersion = 1;
constexpr size_t kHeaderSize = 24;

struct Crc32Table {
  uint32_t t[256];
  Crc32Table() {
    for (uint32_t i = 0; i < 256; ++i) {
      uint32_t c = i;
      for (int k = 0; k < 8; ++k) c = (c & 1) ? (0xEDB88320u ^ (c >> 1)) : (c >> 1);
      t[i] = c;
    }
  }
};

inline void put_u8(std::vector<uint8_t>& o, uint8_t v) { o.push_back(v); }
inline void put_u32(std::vector<uint8_t>& o, uint32_t v) {
  for (int i = 0; i < 4; ++i) o.push_back((uint8_t)(v >> (8 * i)));
}
inline void put_u64(std::vector<uint8_t>& o, uint64_t v) {
  for (int i = 0; i < 8; ++i) o.push_back((uint8_t)(v >> (8 * i)));
}
inline void put_f32s(std::vector<uint8_t>& o, const float* v, size_t n) {
  const size_t at = o.size();
  o.resize(at + 4 * n);
  std::memcpy(o.data() + at, v, 4 * n);  // little-endian host
}

// bincode SerializableVector { id: u64, data: Vec<f32> }
inline void put_vector(std::vector<uint8_t>& o, uint64_t id, const float* v, size_t n) {
  put_u64(o, id);
  put_u64(o, n);
  put_f32s(o, v, n);
}

struct Reader {
  const uint8_t* p;
  size_t n, at = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || n - at < k) {
      ok = false;
      return false;
    }
    return true;
  }
  uint8_t u8() {
    if (!need(1)) return 0;
    return p[at++];
  }
  uint32_t u32() {
    if (!need(4)) return 0;
    uint32_t v = 0;
    for (int i = 0; i < 4; ++i) v |= (uint32_t)p[at + i] << (8 * i);
    at += 4;
    return v;
  }
  uint64_t u64() {
    if (!need(8)) return 0;
    uint64_t v = 0;
    for (int i = 0; i < 8; ++i) v |= (uint64_t)p[at + i] << (8 * i);
    at += 8;
    return v;
  }
  // a sequence length whose elements need at least `elem` bytes each
  uint64_t len(size_t elem) {
    uint64_t v = u64();
    if (ok && elem > 0 && v > (n - at) / elem) ok = false;
    return ok ? v : 0;
  }
  bool f32s(float* dst, size_t cnt) {
    if (!need(4 * cnt)) return false;
    std::memcpy(dst, p + at, 4 * cnt);
    at += 4 * cnt;
    return true;
  }
};

IoResult fail(int status, const std::string& msg) { return IoResult{status, msg}; }

// bincode SerializableVector; appends data to `out`, checks the length
bool read_vector(Reader& r, std::vector<float>& out, uint64_t expect_len, uint64_t* id_out) {
  uint64_t id = r.u64();
  uint64_t len = r.len(4);
  if (!r.ok || len != expect_len) return false;
  size_t at = out.size();
  out.resize(at + len);
  if (!r.f32s(out.data() + at, len)) return false;
  if (id_out) *id_out = id;
  return true;
}

}  // namespace

uint32_t crc32_ieee(const uint8_t* data, size_t n) {
  static const Crc32Table tab;
  uint32_t c = 0xFFFFFFFFu;
  for (size_t i = 0; i < n; ++i) c = tab.t[(c ^ data[i]) & 0xFFu] ^ (c >> 8);
  return c ^ 0xFFFFFFFFu;
}

MappedFile::~MappedFile() {
  if (base_) ::munmap(base_, size_);
}

// Persistable::load_mmap (persistence/mod.rs:70-73, ivf_pq.rs:1983-1993): the
// payload is decoded straight from a read-only private mapping, so a load
// holds no second copy of the file in host memory.
IoResult map_file(const std::string& path, MappedFile& out) {
  int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(FDB_ERR_IO, "cannot open " + path);
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size < 0) {
    ::close(fd);
    return fail(FDB_ERR_IO, "cannot size " + path);
  }
  const size_t sz = (size_t)st.st_size;
  void* p = nullptr;
  if (sz) {
    p = ::mmap(nullptr, sz, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      ::close(fd);
      return fail(FDB_ERR_IO, "cannot map " + path);
    }
    ::madvise(p, sz, MADV_SEQUENTIAL);  // one front-to-back pass: CRC, then decode
  }
  ::close(fd);  // the mapping stays valid after the descriptor closes
  out.base_ = p;
  out.size_ = sz;
  return {};
}

// write_with_header, persistence/mod.rs:169-188 (the disk-space pre-check is
// left to the filesystem: a failed write reports FDB_ERR_IO).
IoResult write_file(const std::string& path, IndexType type, const std::vector<uint8_t>& payload) {
  std::vector<uint8_t> hdr;
  hdr.insert(hdr.end(), kMagic, kMagic + 8);
  put_u32(hdr, kFormatVersion);
  put_u32(hdr, (uint32_t)type);
  put_u32(hdr, 0);  // flags: every reference write path leaves them clear
  put_u32(hdr, crc32_ieee(payload.data(), payload.size()));
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f) return fail(FDB_ERR_IO, "cannot create " + path);
  bool ok = std::fwrite(hdr.data(), 1, hdr.size(), f) == hdr.size();
  ok = ok && (payload.empty() || std::fwrite(payload.data(), 1, payload.size(), f) == payload.size());
  ok = (std::fclose(f) == 0) && ok;
  if (!ok) return fail(FDB_ERR_IO, "write failed on " + path);
  return {};
}

// verify_header, persistence/mod.rs:77-94 with FileHeader::from_bytes/verify,
// format.rs:133-184.
IoResult verify_header(const uint8_t* file, size_t n, IndexType expected, size_t& payload_off) {
  if (n < kHeaderSize) return fail(FDB_ERR_INVALID_FORMAT, "file too small for header");
  if (std::memcmp(file, kMagic, 8) != 0)
    return fail(FDB_ERR_INVALID_FORMAT, "invalid magic bytes");
  Reader r{file + 8, 16};
  uint32_t version = r.u32();
  uint32_t type = r.u32();
  (void)r.u32();  // flags
  uint32_t checksum = r.u32();
  if (type < 1 || type > 4) return fail(FDB_ERR_INVALID_FORMAT, "unknown index type");
  if (version > kFormatVersion)
    return fail(FDB_ERR_INVALID_FORMAT, "unsupported version " + std::to_string(version));
  if (type != (uint32_t)expected) return fail(FDB_ERR_INVALID_FORMAT, "index type mismatch");
  if (crc32_ieee(file + kHeaderSize, n - kHeaderSize) != checksum)
    return fail(FDB_ERR_CHECKSUM_MISMATCH, "checksum mismatch");
  payload_off = kHeaderSize;
  return {};
}

// SerializableIVFPQ field order (ivf_pq.rs:307-316): centroids, pq
// {codebooks, n_subvectors, subvector_dim, dim}, partitions [{ids, codes}],
// nprobe, metric, original_vectors, rerank_factor.
// original_vectors holds one record per id that has an original vector (the
// map's entries; a deleted id has none), at its first entry in list order.
std::vector<uint8_t> encode_ivfpq(const IvfPqArtifacts& a) {
  std::vector<uint8_t> o;
  const uint64_t n = a.ids.size();
  std::vector<uint64_t> rec;  // list positions of the records
  if (a.has_originals) {
    std::unordered_map<uint64_t, bool> seen;
    seen.reserve(n);
    for (uint64_t i = 0; i < n; ++i)
      if (a.orig_ok[i] && seen.emplace(a.ids[i], true).second) rec.push_back(i);
  }
  o.reserve(64 + a.centroids.size() * 4 + a.codebooks.size() * 4 + n * (8 + 8 + a.M) +
            a.nlist * 16 + rec.size() * (16 + 4 * a.dim));
  put_u64(o, a.nlist);
  for (uint32_t c = 0; c < a.nlist; ++c) put_vector(o, c, &a.centroids[(size_t)c * a.dim], a.dim);
  put_u64(o, a.M);
  for (uint32_t m = 0; m < a.M; ++m) {
    put_u64(o, 256);
    for (int j = 0; j < 256; ++j)
      put_vector(o, (uint64_t)j, &a.codebooks[((size_t)m * 256 + j) * a.dsub], a.dsub);
  }
  put_u64(o, a.M);
  put_u64(o, a.dsub);
  put_u64(o, a.dim);
  put_u64(o, a.nlist);
  for (uint32_t l = 0; l < a.nlist; ++l) {
    const uint64_t s = a.offsets[l], e = a.offsets[l + 1];
    put_u64(o, e - s);
    for (uint64_t i = s; i < e; ++i) put_u64(o, a.ids[i]);
    put_u64(o, e - s);
    for (uint64_t i = s; i < e; ++i) {
      put_u64(o, a.M);
      o.insert(o.end(), a.codes.begin() + i * a.M, a.codes.begin() + (i + 1) * a.M);
    }
  }
  put_u64(o, a.nprobe);
  put_u32(o, a.metric);
  if (a.has_originals) {
    put_u8(o, 1);
    put_u64(o, rec.size());
    for (uint64_t i : rec) put_vector(o, a.ids[i], &a.originals[i * a.dim], a.dim);
  } else {
    put_u8(o, 0);
  }
  put_u64(o, a.rerank_factor);
  return o;
}

IoResult decode_ivfpq(const uint8_t* p, size_t n, IvfPqArtifacts& a) {
  Reader r{p, n};
  const std::string bad = "bincode: malformed IVF-PQ payload";
  uint64_t nlist = r.len(16);
  if (!r.ok || nlist == 0 || nlist > 0xFFFFFFFFull) return fail(FDB_ERR_INVALID_FORMAT, bad);
  // the first centroid fixes the dimension
  uint64_t dim = 0;
  a.centroids.clear();
  for (uint64_t c = 0; c < nlist; ++c) {
    uint64_t id = r.u64();
    (void)id;
    uint64_t len = r.len(4);
    if (!r.ok) return fail(FDB_ERR_INVALID_FORMAT, bad);
    if (c == 0) {
      dim = len;
      if (dim == 0 || dim > 0xFFFFFFFFull) return fail(FDB_ERR_INVALID_FORMAT, "zero dimension");
      // every centroid record takes 16 + 4*dim bytes: check before reserving
      if (nlist > (r.n - r.at + 16) / (16 + 4 * dim)) return fail(FDB_ERR_INVALID_FORMAT, bad);
      a.centroids.reserve(nlist * dim);
    } else if (len != dim) {
      return fail(FDB_ERR_INVALID_FORMAT, "centroid dimensions differ");
    }
    size_t at = a.centroids.size();
    a.centroids.resize(at + len);
    if (!r.f32s(a.centroids.data() + at, len)) return fail(FDB_ERR_INVALID_FORMAT, bad);
  }
  uint64_t M = r.len(8);
  if (!r.ok || M == 0 || dim % M != 0) return fail(FDB_ERR_INVALID_FORMAT, "bad codebook count");
  const uint64_t dsub = dim / M;
  a.codebooks.clear();
  if (M > (r.n - r.at) / (8 + 256 * (16 + 4 * dsub))) return fail(FDB_ERR_INVALID_FORMAT, bad);
  a.codebooks.reserve(M * 256 * dsub);
  for (uint64_t m = 0; m < M; ++m) {
    uint64_t kc = r.len(16);
    if (!r.ok) return fail(FDB_ERR_INVALID_FORMAT, bad);
    if (kc != 256) return fail(FDB_ERR_UNSUPPORTED, "codebooks must hold 256 centroids");
    for (uint64_t j = 0; j < kc; ++j)
      if (!read_vector(r, a.codebooks, dsub, nullptr))
        return fail(FDB_ERR_INVALID_FORMAT, "codebook vector of the wrong length");
  }
  uint64_t n_sub = r.u64(), sub_dim = r.u64(), pq_dim = r.u64();
  if (!r.ok || n_sub != M || sub_dim != dsub || pq_dim != dim)
    return fail(FDB_ERR_INVALID_FORMAT, "PQ shape disagrees with its codebooks");
  uint64_t nparts = r.len(16);
  if (!r.ok || nparts != nlist) return fail(FDB_ERR_INVALID_FORMAT, "partition count != nlist");
  a.offsets.assign(1, 0);
  a.ids.clear();
  a.codes.clear();
  for (uint64_t l = 0; l < nparts; ++l) {
    uint64_t ni = r.len(8);
    if (!r.ok) return fail(FDB_ERR_INVALID_FORMAT, bad);
    size_t at = a.ids.size();
    a.ids.resize(at + ni);
    for (uint64_t i = 0; i < ni; ++i) a.ids[at + i] = r.u64();
    uint64_t nc = r.len(8 + M);
    if (!r.ok || nc != ni) return fail(FDB_ERR_INVALID_FORMAT, "partition ids/codes differ in length");
    for (uint64_t i = 0; i < nc; ++i) {
      uint64_t cl = r.len(1);
      if (!r.ok || cl != M) return fail(FDB_ERR_INVALID_FORMAT, "code of the wrong length");
      if (!r.need(M)) return fail(FDB_ERR_INVALID_FORMAT, bad);
      a.codes.insert(a.codes.end(), p + r.at, p + r.at + M);
      r.at += M;
    }
    a.offsets.push_back(a.ids.size());
  }
  a.nprobe = r.u64();
  uint32_t metric = r.u32();
  if (!r.ok || metric > 4) return fail(FDB_ERR_INVALID_FORMAT, "bad metric");
  uint8_t tag = r.u8();
  if (!r.ok || tag > 1) return fail(FDB_ERR_INVALID_FORMAT, "bad Option tag");
  a.has_originals = false;
  a.originals.clear();
  a.orig_ok.clear();
  if (tag == 1) {
    uint64_t nv = r.len(16);
    if (!r.ok || nv > (r.n - r.at) / (16 + 4 * dim)) return fail(FDB_ERR_INVALID_FORMAT, bad);
    // from_serializable (ivf_pq.rs:1918-1925) collects the records into a
    // map: a later record of an id replaces an earlier one
    std::unordered_map<uint64_t, uint64_t> where;
    std::vector<float> vecs;
    vecs.reserve(nv * dim);
    for (uint64_t i = 0; i < nv; ++i) {
      uint64_t id;
      if (!read_vector(r, vecs, dim, &id)) return fail(FDB_ERR_INVALID_FORMAT, bad);
      where[id] = i;
    }
    // an entry whose id has no record (the reference's delete removes the
    // id's vector but saves the entry, tombstones being unsaved) has no
    // original; reranking drops it (filter_map, ivf_pq.rs:562-571).
    // Records of ids no list holds are not kept.
    const uint64_t N = a.ids.size();
    a.originals.assign(N * dim, 0.0f);
    a.orig_ok.assign(N, 0);
    for (uint64_t i = 0; i < N; ++i) {
      auto it = where.find(a.ids[i]);
      if (it == where.end()) continue;
      std::memcpy(&a.originals[i * dim], &vecs[it->second * dim], 4 * dim);
      a.orig_ok[i] = 1;
    }
    a.has_originals = true;
  }
  a.rerank_factor = r.u64();
  if (!r.ok) return fail(FDB_ERR_INVALID_FORMAT, bad);
  a.nlist = (uint32_t)nlist;
  a.dim = (uint32_t)dim;
  a.M = (uint32_t)M;
  a.dsub = (uint32_t)dsub;
  a.metric = metric;
  return {};
}

std::vector<uint8_t> encode_bf(const BruteForceArtifacts& a) {
  std::vector<uint8_t> o;
  o.reserve(17 + a.n * 8 + a.n * a.dim * 4);
  put_u8(o, (uint8_t)a.metric);
  put_u64(o, a.n);
  put_u64(o, a.dim);
  for (uint64_t i = 0; i < a.n; ++i) put_u64(o, a.ids[i]);
  put_f32s(o, a.data.data(), a.n * a.dim);
  return o;
}

// BruteForceIndex::load, brute_force.rs:323-384
IoResult decode_bf(const uint8_t* p, size_t n, BruteForceArtifacts& a) {
  if (n < 17) return fail(FDB_ERR_INVALID_FORMAT, "brute-force payload too small");
  Reader r{p, n};
  uint8_t metric = r.u8();
  if (metric > 4) return fail(FDB_ERR_INVALID_FORMAT, "unknown metric byte");
  uint64_t cnt = r.u64(), dim = r.u64();
  uint64_t rem = n - 17;
  if (cnt > rem / 8) return fail(FDB_ERR_INVALID_FORMAT, "brute-force payload truncated");
  rem -= cnt * 8;
  if (cnt && dim > rem / 4 / cnt) return fail(FDB_ERR_INVALID_FORMAT, "brute-force payload truncated");
  a.metric = metric;
  a.n = cnt;
  a.dim = dim;
  a.ids.resize(cnt);
  for (uint64_t i = 0; i < cnt; ++i) a.ids[i] = r.u64();
  a.data.resize(cnt * dim);
  r.f32s(a.data.data(), cnt * dim);
  return {};
}

}  // namespace fdb
