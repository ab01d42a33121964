// Native GGUF reader (src/gguf/reader.js:136-190, type table src/gguf/types.js:24-65).
#include "gguf.h"

#include <stdio.h>
#include <string.h>

#include "zl_common.h"

namespace zl {

namespace {
struct TypeInfo { int block, bytes; };
TypeInfo type_info(int t) {
  switch (t) {
    case 0: return {1, 4}; case 1: return {1, 2}; case 2: return {32, 18}; case 3: return {32, 20};
    case 6: return {32, 22}; case 7: return {32, 24}; case 8: return {32, 34}; case 9: return {32, 36};
    case 10: return {256, 84}; case 11: return {256, 110}; case 12: return {256, 144}; case 13: return {256, 176};
    case 14: return {256, 210}; case 15: return {256, 292}; case 16: return {256, 66}; case 17: return {256, 74};
    case 18: return {256, 98}; case 19: return {256, 50}; case 20: return {32, 18}; case 21: return {256, 110};
    case 22: return {256, 82}; case 23: return {256, 136}; case 24: return {1, 1}; case 25: return {1, 2};
    case 26: return {1, 4}; case 27: return {1, 8}; case 28: return {1, 8}; case 29: return {256, 56}; case 30: return {1, 2};
    default: return {0, 0};
  }
}

struct Cursor {
  FILE *f;
  uint64_t size, pos = 0;
  void take(void *dst, uint64_t n) {
    if (pos + n > size)
      throw Error(ZL_ERR_FORMAT, "GGUF: unexpected end of file at byte " + std::to_string(pos) + " (need " + std::to_string(n) +
                                     " more, file is " + std::to_string(size) + " bytes)");
    if (fread(dst, 1, n, f) != n) throw Error(ZL_ERR_IO, "GGUF: short read");
    pos += n;
  }
  template <typename T> T get() { T v; take(&v, sizeof(T)); return v; }
  std::string str() {
    uint64_t n = get<uint64_t>();
    if (n > (1u << 30)) throw Error(ZL_ERR_FORMAT, "GGUF: implausible string length " + std::to_string(n));
    std::string s(n, '\0');
    if (n) take(&s[0], n);
    return s;
  }
};

double scalar(Cursor &c, int t) {
  switch (t) {
    case 0: return c.get<uint8_t>(); case 1: return c.get<int8_t>(); case 2: return c.get<uint16_t>();
    case 3: return c.get<int16_t>(); case 4: return c.get<uint32_t>(); case 5: return c.get<int32_t>();
    case 6: return c.get<float>(); case 7: return c.get<uint8_t>() != 0; case 10: return (double)c.get<uint64_t>();
    case 11: return (double)c.get<int64_t>(); case 12: return c.get<double>();
    default: throw Error(ZL_ERR_FORMAT, "GGUF: unknown metadata value type " + std::to_string(t));
  }
}

void read_value(Cursor &c, int t, GGUFValue &v) {
  v.type = t;
  if (t == 8) { v.str = c.str(); return; }
  if (t == 9) {
    int et = (int)c.get<uint32_t>();
    uint64_t n = c.get<uint64_t>();
    if (n > (1u << 28)) throw Error(ZL_ERR_FORMAT, "GGUF: implausible array length " + std::to_string(n));
    v.arrLen = n;
    for (uint64_t i = 0; i < n; i++) {
      if (et == 8) c.str();
      else if (et == 9) { GGUFValue sub; read_value(c, 9, sub); (void)sub; }
      else v.arr.push_back(scalar(c, et));
    }
    return;
  }
  v.num = scalar(c, t);
}
}  // namespace

int ggml_block_size(int type) { return type_info(type).block; }

int64_t ggml_row_bytes(int type, int64_t cols) {
  TypeInfo ti = type_info(type);
  if (!ti.block) return -1;
  if (cols % ti.block) return -1;
  return cols / ti.block * ti.bytes;
}

GGUF read_gguf(const std::string &path) {
  FILE *f = fopen(path.c_str(), "rb");
  if (!f) throw Error(ZL_ERR_IO, "cannot open " + path);
  GGUF g;
  g.path = path;
  try {
    fseek(f, 0, SEEK_END);
    g.fileSize = (uint64_t)ftell(f);
    fseek(f, 0, SEEK_SET);
    Cursor c{f, g.fileSize};
    char magic[4];
    c.take(magic, 4);
    if (memcmp(magic, "GGUF", 4) != 0) throw Error(ZL_ERR_FORMAT, "not a GGUF file");
    g.version = c.get<uint32_t>();
    if (g.version < 2 || g.version > 3) throw Error(ZL_ERR_FORMAT, "unsupported GGUF version " + std::to_string(g.version) + " (expected 2 or 3)");
    uint64_t nt = c.get<uint64_t>(), nkv = c.get<uint64_t>();
    if (nt > 1000000 || nkv > 1000000) throw Error(ZL_ERR_FORMAT, "GGUF: implausible tensor/metadata count (corrupt file?)");
    for (uint64_t i = 0; i < nkv; i++) {
      std::string key = c.str();
      int t = (int)c.get<uint32_t>();
      GGUFValue v;
      read_value(c, t, v);
      g.meta[key] = v;
    }
    double al = g.num("general.alignment", 32);
    if (al <= 0 || al != (double)(uint32_t)al) throw Error(ZL_ERR_FORMAT, "GGUF: bad general.alignment");
    g.alignment = (uint32_t)al;
    for (uint64_t i = 0; i < nt; i++) {
      GGUFTensor t;
      t.name = c.str();
      uint32_t nd = c.get<uint32_t>();
      if (nd < 1 || nd > 8) throw Error(ZL_ERR_FORMAT, "GGUF: tensor " + t.name + " has " + std::to_string(nd) + " dims");
      for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.get<uint64_t>());
      t.type = (int)c.get<uint32_t>();
      t.offset = c.get<uint64_t>();
      g.index[t.name] = g.tensors.size();
      g.tensors.push_back(t);
    }
    g.dataStart = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
    for (auto &t : g.tensors) {
      t.absOffset = g.dataStart + t.offset;
      uint64_t rows = 1;
      for (size_t d = 1; d < t.dims.size(); d++) rows *= t.dims[d];
      int64_t rb = ggml_row_bytes(t.type, (int64_t)t.dims[0]);
      t.nBytes = rb < 0 ? 0 : (uint64_t)rb * rows;
      if (rb >= 0 && t.absOffset + t.nBytes > g.fileSize)
        throw Error(ZL_ERR_FORMAT, "GGUF: tensor " + t.name + " extends past end of file (truncated download?)");
    }
  } catch (...) {
    fclose(f);
    throw;
  }
  fclose(f);
  return g;
}

}  // namespace zl
