// NETW v1 weight files (serialization::save_parameters / load_parameters,
// serialization.cpp:8-111, reached through Layer::save_weights /
// load_weights, layer.cpp:463-470) written from and read into the device
// decoder, over TransformerDecoder::parameters() order (layer.cpp:
// 1140-1154).  Layout, little-endian: "NETW", uint16 version 1, uint32
// tensor count, then per tensor uint32 rank, uint64 extent per dimension,
// uint64 element count and the fp32 elements in row-major order.
#include "engine.hpp"

#include <cstdint>
#include <fstream>
#include <string>
#include <vector>

namespace nnhip {

// The reference's shape of parameters()[idx]: Embedding weight [V][d]
// (layer.cpp:267-268), Dense weight [in][out] and bias [1][out]
// (layer.cpp:153-157), LayerNorm gamma / beta Shape{embed_dim}
// (layer.cpp:204-209, 1063-1064).
std::vector<uint64_t> param_dims(const Model &m, int idx) {
  int64_t r = 0, c = 0;
  m.param_shape(idx, &r, &c);
  const int last = 1 + 18 * m.L;
  const bool norm = idx >= 1 && idx < last && (idx - 1) % 18 >= 14;
  if (norm) return {(uint64_t)c};
  return {(uint64_t)r, (uint64_t)c};
}

void save_weights(const Model &m, const std::string &path) {
  std::ofstream out(path, std::ios::binary);
  NNHIP_REQUIRE((bool)out, kErrIO, "Failed to open file for writing: " + path);
  out.write("NETW", 4);
  const uint16_t version = 1;
  out.write(reinterpret_cast<const char *>(&version), sizeof(version));
  const uint32_t count = (uint32_t)m.num_params();
  out.write(reinterpret_cast<const char *>(&count), sizeof(count));
  std::vector<float> host;
  for (int i = 0; i < m.num_params(); ++i) {
    const std::vector<uint64_t> dims = param_dims(m, i);
    const uint32_t rank = (uint32_t)dims.size();
    out.write(reinterpret_cast<const char *>(&rank), sizeof(rank));
    uint64_t n = 1;
    for (uint64_t e : dims) {
      out.write(reinterpret_cast<const char *>(&e), sizeof(e));
      n *= e;
    }
    out.write(reinterpret_cast<const char *>(&n), sizeof(n));
    host.resize(n);
    m.get_param(i, host.data());
    out.write(reinterpret_cast<const char *>(host.data()),
              (std::streamsize)(n * sizeof(float)));
  }
  out.flush();
  NNHIP_REQUIRE((bool)out, kErrIO, "Failed to write file: " + path);
}

void load_weights(Model &m, const std::string &path) {
  std::ifstream in(path, std::ios::binary);
  NNHIP_REQUIRE((bool)in, kErrIO, "Failed to open file for reading: " + path);
  // a read that comes up short is reported (the reference does not check)
  auto rd = [&](void *p, size_t bytes) {
    in.read(reinterpret_cast<char *>(p), (std::streamsize)bytes);
    NNHIP_REQUIRE((size_t)in.gcount() == bytes, kErrArg,
                  "Unexpected end of file: " + path);
  };
  char magic[4];
  in.read(magic, 4);
  NNHIP_REQUIRE(in.gcount() == 4 && std::string(magic, 4) == "NETW", kErrArg,
                "Invalid file format signature.");
  uint16_t version = 0;
  rd(&version, sizeof(version));
  NNHIP_REQUIRE(version == 1, kErrArg,
                "Unsupported serialization file version: " + std::to_string(version));
  uint32_t count = 0;
  rd(&count, sizeof(count));
  NNHIP_REQUIRE(count == (uint32_t)m.num_params(), kErrArg,
                "Tensor count mismatch (file has " + std::to_string(count) +
                    ", model has " + std::to_string(m.num_params()) + ").");
  std::vector<float> host;
  for (int i = 0; i < m.num_params(); ++i) {
    const std::vector<uint64_t> dims = param_dims(m, i);
    uint32_t rank = 0;
    rd(&rank, sizeof(rank));
    NNHIP_REQUIRE(rank == dims.size(), kErrArg, "Tensor dimension count mismatch.");
    uint64_t n = 1;
    for (size_t d = 0; d < dims.size(); ++d) {
      uint64_t e = 0;
      rd(&e, sizeof(e));
      NNHIP_REQUIRE(e == dims[d], kErrArg,
                    "Tensor shape mismatch at dimension " + std::to_string(d));
      n *= e;
    }
    uint64_t ne = 0;
    rd(&ne, sizeof(ne));
    NNHIP_REQUIRE(ne == n, kErrArg, "Tensor element count mismatch.");
    host.resize(n);
    rd(host.data(), n * sizeof(float));
    m.set_param(i, host.data());
  }
}

}  // namespace nnhip
