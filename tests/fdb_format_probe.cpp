// Test driver for the library's host-side .fdb codec (fdb_format.cpp), built
// with g++ by tests/test_format_host.py: no device is involved.
//   fdb_format_probe <in.fdb> [out.fdb]
// decodes an IVF-PQ file and prints its fields; with out.fdb it writes the
// decoded index back with the library's encoder.
#include <cstdio>

#include "fdb_format.hpp"

int main(int argc, char** argv) {
  if (argc < 2) return 2;
  fdb::MappedFile f;
  fdb::IoResult r = fdb::map_file(argv[1], f);
  size_t off = 0;
  if (r.status == 0) r = fdb::verify_header(f.data(), f.size(), fdb::IndexType::IvfPq, off);
  fdb::IvfPqArtifacts a;
  if (r.status == 0) r = fdb::decode_ivfpq(f.data() + off, f.size() - off, a);
  if (r.status != 0) {
    std::printf("status %d %s\n", r.status, r.message.c_str());
    return 0;
  }
  std::printf("status 0\nnlist %u dim %u M %u n %zu nprobe %llu metric %u rerank_factor %llu originals %d\n",
              a.nlist, a.dim, a.M, a.ids.size(), (unsigned long long)a.nprobe, a.metric,
              (unsigned long long)a.rerank_factor, a.has_originals ? 1 : 0);
  std::printf("orig_ok ");
  for (uint8_t v : a.orig_ok) std::putchar('0' + v);
  std::printf("\n");
  if (argc > 2) {
    r = fdb::write_file(argv[2], fdb::IndexType::IvfPq, fdb::encode_ivfpq(a));
    std::printf("write %d\n", r.status);
  }
  return 0;
}
