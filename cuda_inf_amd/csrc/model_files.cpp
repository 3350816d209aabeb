// Model files on the host side of the attention path: the weight index
// (index.bin), the weight blob's upload into HBM (weights.bin), and the
// byte-level BPE tokenizer.  C-ABI in include/cuda_inf_model.h.
//
// Index and blob: src/engine.cu:55-78 (Model, its name -> tensor lookup),
// 664-692 (reading index.bin, uploading weights.bin); the format is
// tools/make_index.py:3-11.  Tokenizer: src/tokenizer.h (GPT-2 byte-level
// BPE with a hand-written pre-tokenizer).  The tokenizer here keeps the
// reference's observable behaviour (same pieces, same merge order, same
// decoded bytes, including its treatment of malformed UTF-8 and of
// non-ASCII code points as letters) with its own data layout: symbols are
// interned once at load, merges are keyed by symbol-index pairs, special
// tokens are bucketed by first byte and the text is scanned once.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <climits>
#include <memory>
#include <mutex>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "cuda_inf_model.h"

namespace cia {
void set_hip_error(hipError_t e);
}

namespace {

// ---------------------------------------------------------------- files

bool read_file(const char* path, std::string& out) {
  FILE* f = fopen(path, "rb");
  if (!f) return false;
  char buf[1 << 16];
  size_t r;
  out.clear();
  while ((r = fread(buf, 1, sizeof buf, f)) > 0) out.append(buf, r);
  const bool ok = !ferror(f);
  fclose(f);
  return ok;
}

// Reads [off, off + len) of fd into dst with up to kReaders threads (no
// more than the host's hardware threads), each a contiguous slice; false
// on a read error or a file shorter than asked.  Reading from the page
// cache, one thread moves ~8 GB/s: 12 keep the PCIe copies fed (a 2 GiB
// file: 4 readers 32 GB/s, 8 41 GB/s, 12 43-45 GB/s).
constexpr int kReaders = 12;
constexpr uint64_t kSlice = 4ull << 20;  // (no thread gets less than 4 MiB)

bool pread_all(int fd, uint8_t* dst, uint64_t off, uint64_t len) {
  while (len > 0) {
    const ssize_t r = pread(fd, dst, (size_t)std::min<uint64_t>(len, 1ull << 30), (off_t)off);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    dst += r;
    off += (uint64_t)r;
    len -= (uint64_t)r;
  }
  return true;
}

bool read_parallel(int fd, uint8_t* dst, uint64_t off, uint64_t len) {
  static const uint64_t hw = std::max(1u, std::thread::hardware_concurrency());
  const int nt = (int)std::max<uint64_t>(
      1, std::min<uint64_t>(std::min<uint64_t>(kReaders, hw), len / kSlice));
  const uint64_t per = (len + nt - 1) / nt;
  bool ok[kReaders];
  std::thread th[kReaders];
  for (int t = 1; t < nt; t++) {
    const uint64_t a = std::min(len, t * per), b = std::min(len, (t + 1) * per);
    try {
      th[t] = std::thread([=, &ok] { ok[t] = pread_all(fd, dst + a, off + a, b - a); });
    } catch (...) {  // (no thread to be had: this slice on the calling thread)
      ok[t] = pread_all(fd, dst + a, off + a, b - a);
    }
  }
  ok[0] = pread_all(fd, dst, off, std::min(len, per));
  for (int t = 1; t < nt; t++)
    if (th[t].joinable()) th[t].join();
  for (int t = 0; t < nt; t++)
    if (!ok[t]) return false;
  return true;
}

template <typename T>
bool take(const std::string& s, size_t& p, T& v) {
  if (s.size() - p < sizeof(T)) return false;
  memcpy(&v, s.data() + p, sizeof(T));  // (little-endian host, as the file)
  p += sizeof(T);
  return true;
}

// ---------------------------------------------------------------- tokenizer

// UTF-8 length of a lead byte as the reference reads it (tokenizer.h:86,
// 160): 1 for ASCII, 2 for 110xxxxx, 3 for 1110xxxx, else 4 (also for a
// stray continuation byte, so malformed text is consumed 4 bytes at a time)
inline int lead_len(unsigned char c) {
  return c < 0x80 ? 1 : (c >> 5) == 0x6 ? 2 : (c >> 4) == 0xE ? 3 : 4;
}

void put_utf8(uint32_t cp, std::string& o) {
  if (cp < 0x80) {
    o.push_back((char)cp);
  } else if (cp < 0x800) {
    o.push_back((char)(0xC0 | (cp >> 6)));
    o.push_back((char)(0x80 | (cp & 0x3F)));
  } else if (cp < 0x10000) {
    o.push_back((char)(0xE0 | (cp >> 12)));
    o.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
    o.push_back((char)(0x80 | (cp & 0x3F)));
  } else {
    o.push_back((char)(0xF0 | (cp >> 18)));
    o.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
    o.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
    o.push_back((char)(0x80 | (cp & 0x3F)));
  }
}

// code points of s (tokenizer.h:83-92: the lead byte's payload bits, then
// 6 bits of each following byte that exists, whatever its top bits)
void code_points(const char* s, size_t n, std::vector<uint32_t>& cps) {
  cps.clear();
  for (size_t i = 0; i < n;) {
    const unsigned char c = (unsigned char)s[i];
    const int k = lead_len(c);
    uint32_t cp = k == 1 ? c : k == 2 ? (c & 0x1Fu) : k == 3 ? (c & 0xFu) : (c & 0x7u);
    for (int j = 1; j < k && i + j < n; j++) cp = (cp << 6) | ((unsigned char)s[i + j] & 0x3Fu);
    cps.push_back(cp);
    i += (size_t)k;
  }
}

// character classes of the pre-tokenizer (tokenizer.h:93-102): ASCII
// letters and every non-whitespace code point >= 0x80 are letters
enum Cls : uint8_t { kLetter, kDigit, kSpace, kNewline, kOtherWs, kPunct };

inline Cls cls(uint32_t c) {
  if (c == ' ') return kSpace;
  if (c == '\n' || c == '\r') return kNewline;
  if (c == '\t' || c == 0x0b || c == 0x0c || c == 0xa0) return kOtherWs;
  if (c >= '0' && c <= '9') return kDigit;
  if ((c | 32) >= 'a' && (c | 32) <= 'z') return kLetter;
  return c >= 0x80 ? kLetter : kPunct;
}
inline bool is_ws(Cls k) { return k == kSpace || k == kNewline || k == kOtherWs; }

// Piece boundaries of one special-free chunk, in order: the GPT-2 pattern
// as tokenizer.h:105-153 evaluates it (contractions; an optional non-letter,
// non-digit, non-whitespace code point or one space, then letters; 1-3
// digits; an optional space, punctuation, then CR/LF; whitespace up to the
// last CR/LF; whitespace but the last before a non-space; whitespace).
void pieces(const std::vector<uint32_t>& c, std::vector<int>& ends) {
  const int n = (int)c.size();
  std::vector<Cls> k(n);
  for (int i = 0; i < n; i++) k[i] = cls(c[i]);
  auto letters_from = [&](int j) {
    while (j < n && k[j] == kLetter) j++;
    return j;
  };
  auto lower = [](uint32_t x) { return x >= 'A' && x <= 'Z' ? x + 32 : x; };
  ends.clear();
  for (int i = 0; i < n;) {
    int e = -1;
    if (c[i] == '\'' && i + 1 < n) {
      const uint32_t a = lower(c[i + 1]);
      if (a == 's' || a == 't' || a == 'm' || a == 'd') {
        e = i + 2;
      } else if (i + 2 < n) {
        const uint32_t b = lower(c[i + 2]);
        if ((a == 'r' && b == 'e') || (a == 'v' && b == 'e') || (a == 'l' && b == 'l')) e = i + 3;
      }
    }
    if (e < 0) {
      const bool next_letter = i + 1 < n && k[i + 1] == kLetter;
      if (k[i] == kLetter) {
        e = letters_from(i);
      } else if ((k[i] == kPunct || k[i] == kSpace) && next_letter) {
        e = letters_from(i + 1);
      } else if (k[i] == kDigit) {
        e = i + 1;
        while (e < n && e < i + 3 && k[e] == kDigit) e++;
      } else {
        const int p = k[i] == kSpace ? i + 1 : i;
        if (p < n && k[p] == kPunct) {
          e = p + 1;
          while (e < n && k[e] == kPunct) e++;
          while (e < n && k[e] == kNewline) e++;
        } else if (is_ws(k[i])) {
          int w = i, nl = -1;
          for (; w < n && is_ws(k[w]); w++)
            if (k[w] == kNewline) nl = w;
          e = nl >= 0 ? nl + 1 : w == n ? n : w - 1 > i ? w - 1 : w;
        } else {
          e = i + 1;
        }
      }
    }
    ends.push_back(e);
    i = e;
  }
}

struct Merge {
  int32_t rank, out;  // out: symbol index of the merged string
};

// No C++ exception crosses the C ABI: a failed allocation while reading a
// file or tokenizing becomes CIA_ERR_IO.
template <typename F>
int guarded(F&& f) {
  try {
    return f();
  } catch (...) {
    return CIA_ERR_IO;
  }
}

}  // namespace

struct cia_tokenizer {
  // symbols: every string the BPE can hold (vocabulary entries, the 256
  // byte-level characters, merge operands and results), interned once;
  // vid[s] its token id, or INT32_MIN when it is not in the vocabulary
  std::unordered_map<std::string, int32_t> sym;
  std::vector<int32_t> vid;
  std::unordered_map<uint64_t, Merge> merges;  // (left << 32 | right) -> rank, result
  std::string byte_char[256];                  // byte -> its byte-level character (UTF-8)
  std::unordered_map<std::string, uint8_t> char_byte;
  std::vector<std::string> id_str;             // token id -> byte-level string
  std::unordered_map<int32_t, std::string> special_str;
  // special tokens by first byte, longest first (then file order)
  std::vector<std::pair<std::string, int32_t>> special_by_byte[256];

  int32_t intern(const std::string& s) {
    auto it = sym.find(s);
    if (it != sym.end()) return it->second;
    const int32_t x = (int32_t)vid.size();
    sym.emplace(s, x);
    vid.push_back(INT32_MIN);
    return x;
  }

  // the GPT-2 byte <-> character table (printable Latin-1 bytes map to
  // themselves, the other 68 to U+0100.. in byte order; tokenizer.h:30-41)
  void byte_table() {
    int next = 0;
    for (int b = 0; b < 256; b++) {
      const bool keep = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
      std::string s;
      put_utf8(keep ? (uint32_t)b : (uint32_t)(256 + next++), s);
      byte_char[b] = s;
      char_byte[s] = (uint8_t)b;
    }
  }

  // raw bytes of every token whose byte-level string is made of table
  // characters -> its id (a piece is a whole token iff its raw bytes are
  // here); merged pieces already seen, by raw bytes (pieces repeat: words),
  // up to kCacheMax entries, shared by encode calls from several threads
  std::unordered_map<std::string, int32_t> raw_vocab;
  static constexpr size_t kCacheMax = 1 << 16;
  mutable std::mutex cache_mu;
  mutable std::unordered_map<std::string, std::vector<int32_t>> cache;

  // one pre-tokenized piece (byte-level string) -> ids
  void bpe(const std::string& w, std::vector<int32_t>& out) const {
    auto it = sym.find(w);
    if (it != sym.end() && vid[it->second] != INT32_MIN) {
      out.push_back(vid[it->second]);  // the whole piece is a token: no merges
      return;
    }
    std::vector<int32_t> s;
    for (size_t i = 0; i < w.size();) {
      const int k = lead_len((unsigned char)w[i]);
      s.push_back(sym.at(w.substr(i, (size_t)k)));  // (every byte-level character is interned)
      i += (size_t)k;
    }
    while (s.size() > 1) {
      int32_t best = INT32_MAX;
      size_t at = 0;
      int32_t res = -1;
      for (size_t j = 0; j + 1 < s.size(); j++) {
        auto m = merges.find((uint64_t)(uint32_t)s[j] << 32 | (uint32_t)s[j + 1]);
        if (m != merges.end() && m->second.rank < best) {
          best = m->second.rank;
          at = j;
          res = m->second.out;
        }
      }
      if (res < 0) break;
      s[at] = res;
      s.erase(s.begin() + (ptrdiff_t)at + 1);
    }
    for (int32_t x : s)
      if (vid[x] != INT32_MIN) out.push_back(vid[x]);
  }

  void encode_chunk(const char* t, size_t n, std::vector<int32_t>& out) const {
    std::vector<uint32_t> cps;
    std::vector<int> ends;
    code_points(t, n, cps);
    pieces(cps, ends);
    // the chunk re-encoded from its code points (the text itself when it is
    // valid UTF-8) and each code point's offset in it
    std::string renc;
    std::vector<uint32_t> off(cps.size() + 1);
    for (size_t i = 0; i < cps.size(); i++) {
      off[i] = (uint32_t)renc.size();
      put_utf8(cps[i], renc);
    }
    off[cps.size()] = (uint32_t)renc.size();
    std::string raw, bl;
    int a = 0;
    for (int e : ends) {
      raw.assign(renc, off[a], off[e] - off[a]);
      a = e;
      // a whole-piece token, or a piece merged before: no byte-level string
      auto v = raw_vocab.find(raw);
      if (v != raw_vocab.end()) {
        out.push_back(v->second);
        continue;
      }
      {
        std::lock_guard<std::mutex> g(cache_mu);
        auto c = cache.find(raw);
        if (c != cache.end()) {
          out.insert(out.end(), c->second.begin(), c->second.end());
          continue;
        }
      }
      bl.clear();
      for (unsigned char b : raw) bl += byte_char[b];
      const size_t first = out.size();
      bpe(bl, out);
      std::lock_guard<std::mutex> g(cache_mu);
      if (cache.size() < kCacheMax)
        cache.emplace(raw, std::vector<int32_t>(out.begin() + (ptrdiff_t)first, out.end()));
    }
  }

  void encode(const char* t, size_t n, std::vector<int32_t>& out) const {
    size_t chunk = 0;
    for (size_t p = 0; p < n;) {
      const std::pair<std::string, int32_t>* hit = nullptr;
      for (const auto& sp : special_by_byte[(unsigned char)t[p]])
        if (sp.first.size() <= n - p && memcmp(t + p, sp.first.data(), sp.first.size()) == 0) {
          hit = &sp;
          break;
        }
      if (!hit) {
        p++;
        continue;
      }
      if (p > chunk) encode_chunk(t + chunk, p - chunk, out);
      out.push_back(hit->second);
      p += hit->first.size();
      chunk = p;
    }
    if (n > chunk) encode_chunk(t + chunk, n - chunk, out);
  }

  // byte-level string -> bytes, character by character (characters outside
  // the table are dropped; tokenizer.h:212-217)
  void flush(std::string& bl, std::string& out) const {
    for (size_t i = 0; i < bl.size();) {
      const int k = lead_len((unsigned char)bl[i]);
      auto it = char_byte.find(bl.substr(i, (size_t)k));
      if (it != char_byte.end()) out.push_back((char)it->second);
      i += (size_t)k;
    }
    bl.clear();
  }

  void decode(const int32_t* ids, int64_t n, bool skip_special, std::string& out) const {
    std::string bl;
    for (int64_t i = 0; i < n; i++) {
      auto s = special_str.find(ids[i]);
      if (s != special_str.end()) {
        flush(bl, out);
        if (!skip_special) out += s->second;
      } else if (ids[i] >= 0 && (size_t)ids[i] < id_str.size()) {
        bl += id_str[(size_t)ids[i]];
      }
    }
    flush(bl, out);
  }
};

namespace {

// lines of a TSV file, trailing '\n' dropped (tokenizer.h:48-50)
bool tsv_lines(const std::string& path, std::vector<std::string>& lines) {
  std::string s;
  if (!read_file(path.c_str(), s)) return false;
  lines.clear();
  for (size_t a = 0; a < s.size();) {
    size_t b = s.find('\n', a);
    if (b == std::string::npos) b = s.size();
    lines.emplace_back(s, a, b - a);
    a = b + 1;
  }
  return true;
}

}  // namespace

extern "C" int cia_index_read(const char* path, cia_tensor_desc* out, int64_t cap,
                              int64_t* count) {
  return guarded([&]() -> int {
    if (!path || !count) return CIA_ERR_NULL;
    std::string s;
    if (!read_file(path, s)) return CIA_ERR_IO;
    size_t p = 0;
    uint32_t nt;
    if (!take(s, p, nt)) return CIA_ERR_IO;
    if (out && cap < (int64_t)nt) {
      *count = nt;
      return CIA_ERR_ARG;
    }
    for (uint32_t i = 0; i < nt; i++) {
      uint8_t nl, kind;
      cia_tensor_desc d;
      memset(&d, 0, sizeof d);
      if (!take(s, p, nl) || s.size() - p < nl) return CIA_ERR_IO;
      memcpy(d.name, s.data() + p, nl);
      p += nl;
      if (!take(s, p, kind) || kind > 1 || !take(s, p, d.offset) || !take(s, p, d.packed) ||
          !take(s, p, d.scales) || !take(s, p, d.d0) || !take(s, p, d.d1))
        return CIA_ERR_IO;
      d.kind = kind;
      if (out) out[i] = d;
    }
    if (p != s.size()) return CIA_ERR_IO;
    *count = nt;
    return CIA_OK;
  });
}

extern "C" int cia_file_size(const char* path, uint64_t* bytes) {
  if (!path || !bytes) return CIA_ERR_NULL;
  struct stat st;
  if (stat(path, &st) != 0 || !S_ISREG(st.st_mode)) return CIA_ERR_IO;
  *bytes = (uint64_t)st.st_size;
  return CIA_OK;
}

extern "C" int cia_weights_upload(const char* path, void* dst, uint64_t cap, uint64_t* nbytes,
                                  void* stream) {
  if (!path || !dst || !nbytes) return CIA_ERR_NULL;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return CIA_ERR_IO;
  struct stat st;
  if (fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
    close(fd);
    return CIA_ERR_IO;
  }
  const uint64_t size = (uint64_t)st.st_size;
  if (size > cap) {
    close(fd);
    return CIA_ERR_ARG;
  }
  const hipStream_t s = (hipStream_t)stream;
  const uint64_t chunk = std::min<uint64_t>(64ull << 20, std::max<uint64_t>(size, 1));
  uint8_t* buf[2] = {nullptr, nullptr};
  hipEvent_t ev[2] = {nullptr, nullptr};
  int rc = CIA_OK;
  auto hip = [&](hipError_t e) {
    if (e != hipSuccess && rc == CIA_OK) {
      cia::set_hip_error(e);
      rc = CIA_ERR_HIP;
    }
    return e == hipSuccess;
  };
  for (int b = 0; b < 2 && rc == CIA_OK; b++) {
    if (hip(hipHostMalloc((void**)&buf[b], chunk, hipHostMallocDefault)))
      hip(hipEventCreateWithFlags(&ev[b], hipEventDisableTiming));
  }
  // chunk i goes through buffer i & 1: its reads wait for the copy of chunk
  // i - 2 (the buffer's last user), then overlap the copy of chunk i - 1
  for (uint64_t off = 0, i = 0; rc == CIA_OK && off < size; off += chunk, i++) {
    const int b = (int)(i & 1);
    const uint64_t len = std::min(chunk, size - off);
    if (i >= 2 && !hip(hipEventSynchronize(ev[b]))) break;
    if (!read_parallel(fd, buf[b], off, len)) {
      rc = CIA_ERR_IO;
      break;
    }
    if (hip(hipMemcpyAsync((uint8_t*)dst + off, buf[b], len, hipMemcpyHostToDevice, s)))
      hip(hipEventRecord(ev[b], s));
  }
  // every enqueued copy has read its buffer before the buffers are freed
  hip(hipStreamSynchronize(s));
  for (int b = 0; b < 2; b++) {
    if (ev[b]) (void)hipEventDestroy(ev[b]);
    if (buf[b]) (void)hipHostFree(buf[b]);
  }
  close(fd);
  if (rc == CIA_OK) *nbytes = size;
  return rc;
}

extern "C" int cia_tok_load(const char* dir, cia_tokenizer** out) {
  return guarded([&]() -> int {
    if (!dir || !out) return CIA_ERR_NULL;
    *out = nullptr;
    const std::string d(dir);
    std::vector<std::string> voc, mer, spe;
    if (!tsv_lines(d + "/vocab.tsv", voc) || !tsv_lines(d + "/merges.tsv", mer) ||
        !tsv_lines(d + "/special.tsv", spe))
      return CIA_ERR_IO;
    std::unique_ptr<cia_tokenizer> t(new cia_tokenizer());
    t->byte_table();
    for (int b = 0; b < 256; b++) t->intern(t->byte_char[b]);
    // vocabulary "<id>\t<token>": a later line for the same token or id wins
    int32_t maxid = 0;
    std::vector<std::pair<int32_t, std::string>> ent;
    for (const auto& ln : voc) {
      const size_t tab = ln.find('\t');
      if (tab == std::string::npos) continue;
      const int32_t id = (int32_t)atoi(ln.substr(0, tab).c_str());
      ent.emplace_back(id, ln.substr(tab + 1));
      t->vid[(size_t)t->intern(ent.back().second)] = id;
      maxid = std::max(maxid, id);
    }
    t->id_str.assign((size_t)maxid + 1, std::string());
    for (const auto& e : ent)
      if (e.first >= 0) t->id_str[(size_t)e.first] = e.second;
    // merges "<rank>\t<A>\t<B>"
    for (const auto& ln : mer) {
      const size_t t1 = ln.find('\t');
      if (t1 == std::string::npos) continue;
      const size_t t2 = ln.find('\t', t1 + 1);
      if (t2 == std::string::npos) continue;
      const std::string a = ln.substr(t1 + 1, t2 - t1 - 1), b = ln.substr(t2 + 1);
      const int32_t rank = (int32_t)atoi(ln.substr(0, t1).c_str());
      const int32_t ia = t->intern(a), ib = t->intern(b), iab = t->intern(a + b);
      t->merges[(uint64_t)(uint32_t)ia << 32 | (uint32_t)ib] = Merge{rank, iab};
    }
    // special tokens "<id>\t<content>"
    std::vector<std::pair<std::string, int32_t>> sp;
    for (const auto& ln : spe) {
      const size_t tab = ln.find('\t');
      if (tab == std::string::npos) continue;
      const int32_t id = (int32_t)atoi(ln.substr(0, tab).c_str());
      std::string c = ln.substr(tab + 1);
      t->special_str[id] = c;
      if (!c.empty()) sp.emplace_back(std::move(c), id);
    }
    std::stable_sort(sp.begin(), sp.end(),
                     [](const auto& x, const auto& y) { return x.first.size() > y.first.size(); });
    for (auto& x : sp) t->special_by_byte[(unsigned char)x.first[0]].push_back(x);
    for (const auto& e : t->sym) {
      if (t->vid[(size_t)e.second] == INT32_MIN) continue;
      std::string raw;
      bool ok = true;
      for (size_t i = 0; i < e.first.size() && ok;) {
        const int k = lead_len((unsigned char)e.first[i]);
        auto c = t->char_byte.find(e.first.substr(i, (size_t)k));
        ok = c != t->char_byte.end() && i + (size_t)k <= e.first.size();
        if (ok) raw.push_back((char)c->second);
        i += (size_t)k;
      }
      if (ok) t->raw_vocab[raw] = t->vid[(size_t)e.second];
    }
    *out = t.release();
    return CIA_OK;
  });
}

extern "C" void cia_tok_free(cia_tokenizer* tok) { delete tok; }

extern "C" int cia_tok_encode(const cia_tokenizer* tok, const char* text, int64_t len,
                              int32_t* ids, int64_t cap, int64_t* n) {
  return guarded([&]() -> int {
    if (!tok || !n || (!text && len > 0)) return CIA_ERR_NULL;
    if (len < 0) return CIA_ERR_ARG;
    std::vector<int32_t> v;
    tok->encode(text, (size_t)len, v);
    *n = (int64_t)v.size();
    if (!ids) return CIA_OK;
    if (cap < (int64_t)v.size()) return CIA_ERR_ARG;
    if (!v.empty()) memcpy(ids, v.data(), v.size() * sizeof(int32_t));
    return CIA_OK;
  });
}

extern "C" int cia_tok_decode(const cia_tokenizer* tok, const int32_t* ids, int64_t n,
                              int skip_special, char* out, int64_t cap, int64_t* len) {
  return guarded([&]() -> int {
    if (!tok || !len || (!ids && n > 0)) return CIA_ERR_NULL;
    if (n < 0) return CIA_ERR_ARG;
    std::string s;
    tok->decode(ids, n, skip_special != 0, s);
    *len = (int64_t)s.size();
    if (!out) return CIA_OK;
    if (cap < (int64_t)s.size()) return CIA_ERR_ARG;
    if (!s.empty()) memcpy(out, s.data(), s.size());
    return CIA_OK;
  });
}
