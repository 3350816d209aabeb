// TEST INFRASTRUCTURE ONLY: the reference's own tokenizer (src/tokenizer.h,
// a self-contained header), compiled where it lies by oracle/Makefile into
// oracle/_ref/libreftok.so, behind a C ABI so that tests can check the
// oracle (oracle/model_files.py) and the product tokenizer against it.
// Only tests/ load it; it is built only where the reference tree exists.
#include <algorithm>
#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "tokenizer.h"

extern "C" {

void* ref_tok_load(const char* dir) {
  auto* t = new Tokenizer();
  if (!t->load(dir)) {
    delete t;
    return nullptr;
  }
  return t;
}

void ref_tok_free(void* h) { delete static_cast<Tokenizer*>(h); }

// returns the id count; copies at most cap of them
int64_t ref_tok_encode(void* h, const char* text, int64_t len, int32_t* out, int64_t cap) {
  const std::vector<int> v = static_cast<Tokenizer*>(h)->encode(std::string(text, (size_t)len));
  for (size_t i = 0; i < v.size() && (int64_t)i < cap; i++) out[i] = v[i];
  return (int64_t)v.size();
}

// returns the byte count; copies at most cap of them
int64_t ref_tok_decode(void* h, const int32_t* ids, int64_t n, int skip_special, char* out,
                       int64_t cap) {
  const std::vector<int> v(ids, ids + n);
  const std::string s = static_cast<Tokenizer*>(h)->decode(v, skip_special != 0);
  memcpy(out, s.data(), std::min<size_t>(s.size(), (size_t)std::max<int64_t>(cap, 0)));
  return (int64_t)s.size();
}
}
