// .fdb container and payload codecs (host side).
//
// Container (src/persistence/format.rs:82-184, src/persistence/mod.rs:77-94,
// :169-188): 24-byte little-endian header "FORGEDB\0", version u32 (= 1),
// index_type u32 (IvfPq 1, Hnsw 2, Ivf 3, BruteForce 4), flags u32,
// CRC-32/IEEE of the payload u32, then the payload.
//
// IVF-PQ payload: bincode 1.x default encoding (fixed-width little-endian
// integers, u64 sequence lengths, u32 enum variant index, u8 Option tag) of
// SerializableIVFPQ (src/index/ivf_pq.rs:197-328).
//
// Brute-force payload (src/index/brute_force.rs:277-313): metric u8, n u64,
// dim u64, ids [n] u64, data [n*dim] f32.
#pragma once

#include <stdint.h>

#include <string>
#include <vector>

namespace fdb {

enum class IndexType : uint32_t { IvfPq = 1, Hnsw = 2, Ivf = 3, BruteForce = 4 };

uint32_t crc32_ieee(const uint8_t* data, size_t n);

// Flat form of an IVF-PQ index: the layout the device holds.
struct IvfPqArtifacts {
  uint32_t nlist = 0, dim = 0, M = 0, dsub = 0;
  std::vector<float> centroids;     // [nlist][dim]
  std::vector<float> codebooks;     // [M][256][dsub]
  std::vector<uint64_t> offsets;    // [nlist+1]
  std::vector<uint64_t> ids;        // [N]
  std::vector<uint8_t> codes;       // [N][M]
  uint64_t nprobe = 1;
  uint32_t metric = 0;
  bool has_originals = false;
  // original_vectors (ivf_pq.rs:356) is a map id -> vector; here it is held
  // per list entry.  When has_originals: originals [N][dim] in list order and
  // orig_ok [N], 1 where the entry's id has an original vector.  Entries
  // sharing an id share its vector and flag, as map lookups by id would.
  std::vector<float> originals;
  std::vector<uint8_t> orig_ok;
  uint64_t rerank_factor = 1;
};

// Errors are reported as (status, message); status values are fdb_status.
struct IoResult {
  int status = 0;
  std::string message;
};

// A read-only mapping of a whole file, unmapped on destruction.
class MappedFile {
 public:
  MappedFile() = default;
  MappedFile(const MappedFile&) = delete;
  MappedFile& operator=(const MappedFile&) = delete;
  ~MappedFile();
  const uint8_t* data() const { return static_cast<const uint8_t*>(base_); }
  size_t size() const { return size_; }

 private:
  friend IoResult map_file(const std::string& path, MappedFile& out);
  void* base_ = nullptr;
  size_t size_ = 0;
};

// Maps `path` into `out`, which must be empty.
IoResult map_file(const std::string& path, MappedFile& out);
IoResult write_file(const std::string& path, IndexType type, const std::vector<uint8_t>& payload);
// verify_header: returns the payload offset in `file` through payload_off.
IoResult verify_header(const uint8_t* file, size_t n, IndexType expected, size_t& payload_off);

std::vector<uint8_t> encode_ivfpq(const IvfPqArtifacts& a);
IoResult decode_ivfpq(const uint8_t* p, size_t n, IvfPqArtifacts& a);

struct BruteForceArtifacts {
  uint32_t metric = 0;
  uint64_t n = 0, dim = 0;
  std::vector<uint64_t> ids;
  std::vector<float> data;
};
std::vector<uint8_t> encode_bf(const BruteForceArtifacts& a);
IoResult decode_bf(const uint8_t* p, size_t n, BruteForceArtifacts& a);

}  // namespace fdb
