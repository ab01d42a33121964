// Native GGUF reader: header, metadata and tensor infos, as zerollm's readGGUF (src/gguf/reader.js:136-190).
#pragma once
#include <stdint.h>
#include <map>
#include <string>
#include <vector>

namespace zl {

struct GGUFValue {
  int type = -1;        // GGUF value type (src/gguf/types.js:4-7)
  double num = 0;       // numeric scalars and bools
  std::string str;
  std::vector<double> arr;   // numeric arrays
  size_t arrLen = 0;         // length of any array (also string arrays, which are not kept)
};

struct GGUFTensor {
  std::string name;
  std::vector<uint64_t> dims;
  int type = 0;
  uint64_t offset = 0, absOffset = 0, nBytes = 0;
};

struct GGUF {
  std::string path;
  uint64_t fileSize = 0, dataStart = 0;
  uint32_t version = 0, alignment = 32;
  std::map<std::string, GGUFValue> meta;
  std::vector<GGUFTensor> tensors;
  std::map<std::string, size_t> index;

  const GGUFValue *get(const std::string &k) const {
    auto it = meta.find(k);
    return it == meta.end() ? nullptr : &it->second;
  }
  double num(const std::string &k, double dflt) const {
    const GGUFValue *v = get(k);
    return v && v->type != 8 && v->type != 9 ? v->num : dflt;
  }
  const GGUFTensor *tensor(const std::string &n) const {
    auto it = index.find(n);
    return it == index.end() ? nullptr : &tensors[it->second];
  }
};

GGUF read_gguf(const std::string &path);
int64_t ggml_row_bytes(int type, int64_t cols);  // -1 for unknown types
int ggml_block_size(int type);

}  // namespace zl
