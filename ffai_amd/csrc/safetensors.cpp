// safetensors.cpp — the checkpoint reader of libmoehip.so
// (include/moe_safetensors.h).
//
// Format (Sources/FFAI/Loader/SafeTensors.swift:15-31): a little-endian u64
// header length N, N bytes of JSON mapping each tensor name to
// {"dtype", "shape", "data_offsets": [start, end]} (offsets relative to the
// data section at 8 + N), an optional "__metadata__" object, then the raw
// tensor bytes.
//
// Files stay mapped read-only (and open) for the bundle's lifetime. Host reads
// copy out of the mapping. Device uploads are split into chunks that worker
// threads pread straight from the page cache into pinned staging buffers and
// hand to the DMA engine, so filling one chunk overlaps the copy of others and
// no page-table faults are taken on the mapping.
#include <dirent.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <new>
#include <thread>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/moe_safetensors.h"
#include "moe_internal.hpp"

namespace {

moe_status st_fail(moe_status s, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  moe::set_error_text(buf);
  return s;
}

moe_status st_ok() {
  moe::clear_error_text();
  return MOE_OK;
}

#define ST_TRY(expr)                 \
  do {                               \
    moe_status _s = (expr);          \
    if (_s != MOE_OK) return _s;     \
  } while (0)

// ------------------------------------------------------------------ JSON --
// A strict reader for the header and the shard index: objects, arrays,
// strings (with escapes), integers, numbers, true/false/null.
struct JVal {
  enum Kind { NUL, BOOL, INT, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  long long i = 0;
  double d = 0.0;
  std::string s;
  std::vector<JVal> a;
  std::vector<std::pair<std::string, JVal>> o;

  const JVal* get(const char* key) const {
    for (const auto& kv : o)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* p, size_t n) : p_(p), end_(p + n) {}

  bool parse(JVal* out) {
    ws();
    if (!value(out, 0)) return false;
    ws();
    return p_ == end_;
  }

 private:
  const char* p_;
  const char* end_;

  void ws() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  bool lit(const char* w) {
    const size_t n = strlen(w);
    if ((size_t)(end_ - p_) < n || memcmp(p_, w, n) != 0) return false;
    p_ += n;
    return true;
  }
  static void utf8(uint32_t c, std::string* s) {
    if (c < 0x80) {
      s->push_back((char)c);
    } else if (c < 0x800) {
      s->push_back((char)(0xC0 | (c >> 6)));
      s->push_back((char)(0x80 | (c & 0x3F)));
    } else if (c < 0x10000) {
      s->push_back((char)(0xE0 | (c >> 12)));
      s->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (c & 0x3F)));
    } else {
      s->push_back((char)(0xF0 | (c >> 18)));
      s->push_back((char)(0x80 | ((c >> 12) & 0x3F)));
      s->push_back((char)(0x80 | ((c >> 6) & 0x3F)));
      s->push_back((char)(0x80 | (c & 0x3F)));
    }
  }
  bool hex4(uint32_t* v) {
    if (end_ - p_ < 4) return false;
    uint32_t r = 0;
    for (int k = 0; k < 4; k++) {
      const char c = *p_++;
      r <<= 4;
      if (c >= '0' && c <= '9') r |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') r |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') r |= (uint32_t)(c - 'A' + 10);
      else return false;
    }
    *v = r;
    return true;
  }
  bool str(std::string* s) {
    if (p_ >= end_ || *p_ != '"') return false;
    p_++;
    while (p_ < end_) {
      const unsigned char c = (unsigned char)*p_++;
      if (c == '"') return true;
      if (c < 0x20) return false;
      if (c != '\\') {
        s->push_back((char)c);
        continue;
      }
      if (p_ >= end_) return false;
      const char e = *p_++;
      switch (e) {
        case '"': s->push_back('"'); break;
        case '\\': s->push_back('\\'); break;
        case '/': s->push_back('/'); break;
        case 'b': s->push_back('\b'); break;
        case 'f': s->push_back('\f'); break;
        case 'n': s->push_back('\n'); break;
        case 'r': s->push_back('\r'); break;
        case 't': s->push_back('\t'); break;
        case 'u': {
          uint32_t cp;
          if (!hex4(&cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo;
            if (!lit("\\u") || !hex4(&lo) || lo < 0xDC00 || lo >= 0xE000) return false;
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          } else if (cp >= 0xDC00 && cp < 0xE000) {
            return false;
          }
          utf8(cp, s);
          break;
        }
        default: return false;
      }
    }
    return false;
  }
  bool num(JVal* v) {
    const char* s = p_;
    if (p_ < end_ && *p_ == '-') p_++;
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
    if (*p_ == '0') {
      p_++;
    } else {
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    bool integral = true;
    if (p_ < end_ && *p_ == '.') {
      integral = false;
      p_++;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    if (p_ < end_ && (*p_ == 'e' || *p_ == 'E')) {
      integral = false;
      p_++;
      if (p_ < end_ && (*p_ == '+' || *p_ == '-')) p_++;
      if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return false;
      while (p_ < end_ && *p_ >= '0' && *p_ <= '9') p_++;
    }
    const std::string text(s, p_);
    if (integral) {
      errno = 0;
      char* e = nullptr;
      const long long x = strtoll(text.c_str(), &e, 10);
      if (errno == 0 && e && *e == '\0') {
        v->kind = JVal::INT;
        v->i = x;
        v->d = (double)x;
        return true;
      }
    }
    v->kind = JVal::NUM;
    v->d = strtod(text.c_str(), nullptr);
    return true;
  }
  bool value(JVal* v, int depth) {
    if (depth > 64 || p_ >= end_) return false;
    const char c = *p_;
    if (c == '{') {
      p_++;
      v->kind = JVal::OBJ;
      ws();
      if (p_ < end_ && *p_ == '}') {
        p_++;
        return true;
      }
      for (;;) {
        ws();
        std::string key;
        if (!str(&key)) return false;
        ws();
        if (p_ >= end_ || *p_ != ':') return false;
        p_++;
        ws();
        v->o.emplace_back(std::move(key), JVal());
        if (!value(&v->o.back().second, depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          p_++;
          return true;
        }
        return false;
      }
    }
    if (c == '[') {
      p_++;
      v->kind = JVal::ARR;
      ws();
      if (p_ < end_ && *p_ == ']') {
        p_++;
        return true;
      }
      for (;;) {
        ws();
        v->a.emplace_back();
        if (!value(&v->a.back(), depth + 1)) return false;
        ws();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          p_++;
          return true;
        }
        return false;
      }
    }
    if (c == '"') {
      v->kind = JVal::STR;
      return str(&v->s);
    }
    if (lit("true")) {
      v->kind = JVal::BOOL;
      v->b = true;
      return true;
    }
    if (lit("false")) {
      v->kind = JVal::BOOL;
      return true;
    }
    if (lit("null")) return true;
    return num(v);
  }
};

// ----------------------------------------------------------------- dtypes --
// DType.fromSafeTensors (DType.swift:42-55): case-insensitive names.
int st_dtype(const std::string& name, size_t* elsize) {
  std::string u(name);
  for (char& ch : u) ch = (char)toupper((unsigned char)ch);
  static const struct {
    const char* n;
    int dt;
    size_t sz;
  } table[] = {{"F32", MOE_ST_F32, 4}, {"F16", MOE_ST_F16, 2}, {"BF16", MOE_ST_BF16, 2},
               {"I32", MOE_ST_I32, 4}, {"U32", MOE_ST_U32, 4}, {"I64", MOE_ST_I64, 8},
               {"U64", MOE_ST_U64, 8}, {"I8", MOE_ST_I8, 1},   {"U8", MOE_ST_U8, 1}};
  for (const auto& t : table)
    if (u == t.n) {
      *elsize = t.sz;
      return t.dt;
    }
  return -1;
}

// ----------------------------------------------------------------- bundle --
struct MappedFile {
  std::string path;
  int fd = -1;
  void* base = nullptr;
  size_t size = 0;
};

struct Entry {
  int file = 0;
  int dtype = 0;
  std::vector<int64_t> shape;
  size_t offset = 0;  // absolute, in the file
  size_t nbytes = 0;
};

}  // namespace

struct moe_st_bundle {
  std::vector<MappedFile> files;
  std::unordered_map<std::string, Entry> entries;
  std::vector<std::string> names;  // sorted

  ~moe_st_bundle() {
    for (auto& f : files) {
      if (f.base) munmap(f.base, f.size);
      if (f.fd >= 0) close(f.fd);
    }
  }
};

namespace {

bool is_dir(const std::string& p) {
  struct stat sb;
  return stat(p.c_str(), &sb) == 0 && S_ISDIR(sb.st_mode);
}

bool exists(const std::string& p) {
  struct stat sb;
  return stat(p.c_str(), &sb) == 0;
}

bool read_all(const std::string& path, std::string* out) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) return false;
  char buf[65536];
  size_t n;
  while ((n = fread(buf, 1, sizeof(buf), f)) > 0) out->append(buf, n);
  const bool good = !ferror(f);
  fclose(f);
  return good;
}

// SafeTensorsFile.init (SafeTensors.swift:101-230): map the file, parse the
// header, index every entry of a known dtype.
moe_status map_file(moe_st_bundle* b, const std::string& path) {
  if (!exists(path)) return st_fail(MOE_ERR_INVALID, "safetensors file not found: %s", path.c_str());
  char resolved[PATH_MAX];
  if (!realpath(path.c_str(), resolved))
    return st_fail(MOE_ERR_INVALID, "safetensors file not found: %s", path.c_str());
  const int fd = open(resolved, O_RDONLY);
  if (fd < 0) return st_fail(MOE_ERR_INVALID, "mmap failed for %s", resolved);
  struct stat sb;
  if (fstat(fd, &sb) != 0) {
    close(fd);
    return st_fail(MOE_ERR_INVALID, "mmap failed for %s", resolved);
  }
  const size_t size = (size_t)sb.st_size;
  if (size < 8) {
    close(fd);
    return st_fail(MOE_ERR_INVALID, "safetensors header smaller than 8 bytes: %s", resolved);
  }
  void* base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
  if (base == MAP_FAILED) {
    close(fd);
    return st_fail(MOE_ERR_INVALID, "mmap failed for %s", resolved);
  }
  MappedFile mf;
  mf.path = resolved;
  mf.fd = fd;
  mf.base = base;
  mf.size = size;
  b->files.push_back(mf);
  const int fi = (int)b->files.size() - 1;

  const unsigned char* p = static_cast<const unsigned char*>(base);
  uint64_t hlen = 0;
  for (int i = 7; i >= 0; i--) hlen = (hlen << 8) | p[i];
  if (hlen > size - 8)
    return st_fail(MOE_ERR_INVALID, "safetensors JSON header malformed: %s", resolved);
  JVal root;
  JParser jp(reinterpret_cast<const char*>(p + 8), (size_t)hlen);
  if (!jp.parse(&root) || root.kind != JVal::OBJ)
    return st_fail(MOE_ERR_INVALID, "safetensors JSON header malformed: %s", resolved);
  const size_t data_start = 8 + (size_t)hlen;
  for (const auto& kv : root.o) {
    const std::string& name = kv.first;
    if (name == "__metadata__") continue;
    const JVal& v = kv.second;
    const JVal* dt = v.kind == JVal::OBJ ? v.get("dtype") : nullptr;
    const JVal* sh = v.kind == JVal::OBJ ? v.get("shape") : nullptr;
    const JVal* of = v.kind == JVal::OBJ ? v.get("data_offsets") : nullptr;
    if (!dt || dt->kind != JVal::STR || !sh || sh->kind != JVal::ARR || !of ||
        of->kind != JVal::ARR || of->a.size() != 2 || of->a[0].kind != JVal::INT ||
        of->a[1].kind != JVal::INT)
      return st_fail(MOE_ERR_INVALID, "malformed entry for tensor \"%s\"", name.c_str());
    size_t elsize = 0;
    const int dtype = st_dtype(dt->s, &elsize);
    if (dtype < 0) continue;  // not an inference dtype: skipped, as the reference does
    if (sh->a.size() > MOE_ST_MAX_DIMS)
      return st_fail(MOE_ERR_UNSUPPORTED, "tensor \"%s\" has more than %d dimensions",
                     name.c_str(), MOE_ST_MAX_DIMS);
    Entry e;
    e.file = fi;
    e.dtype = dtype;
    unsigned __int128 numel = 1;
    for (const JVal& d : sh->a) {
      if (d.kind != JVal::INT || d.i < 0)
        return st_fail(MOE_ERR_INVALID, "malformed entry for tensor \"%s\"", name.c_str());
      e.shape.push_back(d.i);
      numel *= (unsigned __int128)d.i;
    }
    const long long s0 = of->a[0].i, s1 = of->a[1].i;
    if (s0 < 0 || s1 < s0 || (uint64_t)s1 > size - data_start ||
        numel * elsize != (unsigned __int128)(s1 - s0))
      return st_fail(MOE_ERR_INVALID, "malformed entry for tensor \"%s\"", name.c_str());
    e.offset = data_start + (size_t)s0;
    e.nbytes = (size_t)(s1 - s0);
    b->entries[name] = std::move(e);  // a later shard wins, as in the reference's index
  }
  return MOE_OK;
}

// SafeTensorsBundle.init(directory:) (SafeTensors.swift:248-292).
moe_status bundle_files(const std::string& dir, std::vector<std::string>* out) {
  const std::string index = dir + "/model.safetensors.index.json";
  if (exists(index)) {
    std::string text;
    JVal root;
    if (!read_all(index, &text))
      return st_fail(MOE_ERR_INVALID, "cannot read %s", index.c_str());
    JParser jp(text.data(), text.size());
    const JVal* wm = nullptr;
    if (jp.parse(&root) && root.kind == JVal::OBJ) wm = root.get("weight_map");
    if (!wm || wm->kind != JVal::OBJ)
      return st_fail(MOE_ERR_INVALID, "safetensors JSON header malformed: %s", index.c_str());
    std::vector<std::string> names;
    for (const auto& kv : wm->o) {
      if (kv.second.kind != JVal::STR)
        return st_fail(MOE_ERR_INVALID, "safetensors JSON header malformed: %s", index.c_str());
      names.push_back(kv.second.s);
    }
    std::sort(names.begin(), names.end());
    names.erase(std::unique(names.begin(), names.end()), names.end());
    for (const auto& n : names) out->push_back(dir + "/" + n);
    return MOE_OK;
  }
  const std::string single = dir + "/model.safetensors";
  if (exists(single)) {
    out->push_back(single);
    return MOE_OK;
  }
  DIR* d = opendir(dir.c_str());
  if (!d) return st_fail(MOE_ERR_INVALID, "safetensors file not found: %s", dir.c_str());
  std::vector<std::string> names;
  while (struct dirent* de = readdir(d)) {
    const std::string n = de->d_name;
    const std::string ext = ".safetensors";
    if (n.size() > ext.size() && n.compare(n.size() - ext.size(), ext.size(), ext) == 0)
      names.push_back(n);
  }
  closedir(d);
  std::sort(names.begin(), names.end());
  for (const auto& n : names) out->push_back(dir + "/" + n);
  return MOE_OK;
}

const Entry* find(const moe_st_bundle* b, const char* name) {
  if (!b || !name) return nullptr;
  auto it = b->entries.find(name);
  return it == b->entries.end() ? nullptr : &it->second;
}

moe_status missing(const char* name) {
  return st_fail(MOE_ERR_INVALID, "tensor \"%s\" not present in safetensors bundle",
                 name ? name : "(null)");
}

const unsigned char* entry_bytes(const moe_st_bundle* b, const Entry& e) {
  return static_cast<const unsigned char*>(b->files[e.file].base) + e.offset;
}

moe_status hip_fail(hipError_t e, const char* what) {
  return st_fail(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// Pinned staging shared by every bundle of the process, one set per device:
// kWorkers threads with two kChunk buffers each. The buffers live until the
// process ends (freeing pinned memory during runtime teardown is unsafe).
constexpr int kWorkers = 8;
constexpr size_t kChunk = 8u << 20;

struct Stager {
  void* buf[2 * kWorkers] = {};
  hipEvent_t ev[2 * kWorkers] = {};
  bool ready = false;
};

std::mutex g_stage_mu;  // one upload at a time per process
std::map<int, Stager> g_stagers;

hipError_t stager_init(Stager* S) {
  hipError_t e;
  for (int i = 0; i < 2 * kWorkers; i++) {
    if (!S->buf[i] && (e = hipHostMalloc(&S->buf[i], kChunk, hipHostMallocDefault)) != hipSuccess) {
      S->buf[i] = nullptr;
      return e;
    }
    if (!S->ev[i] && (e = hipEventCreateWithFlags(&S->ev[i], hipEventDisableTiming)) != hipSuccess) {
      S->ev[i] = nullptr;
      return e;
    }
  }
  S->ready = true;
  return hipSuccess;
}

// One contiguous file range and where it goes on the device.
struct Range {
  int fd;
  size_t off, n;
  unsigned char* dst;
};

// File ranges -> device memory. The ranges are cut into kChunk pieces that the
// workers take in order from a shared counter; a worker alternates its two
// buffers: it waits for the buffer's previous DMA, preads the piece into it
// and queues its DMA on `st`. Every worker waits for its last DMAs before
// returning, so the buffers are free afterwards.
moe_status upload_ranges(const std::vector<Range>& rs, hipStream_t st) {
  struct Piece {
    int fd;
    size_t off, n;
    unsigned char* dst;
  };
  std::vector<Piece> pieces;
  for (const Range& r : rs)
    for (size_t o = 0; o < r.n; o += kChunk)
      pieces.push_back({r.fd, r.off + o, std::min(kChunk, r.n - o), r.dst + o});
  if (pieces.empty()) return MOE_OK;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_stage_mu);
  Stager& S = g_stagers[dev];
  if (!S.ready && (e = stager_init(&S)) != hipSuccess) return hip_fail(e, "staging buffers");
  const int P = (int)std::min<size_t>(kWorkers, pieces.size());
  std::atomic<size_t> next{0};
  std::atomic<bool> failed{false};
  std::mutex err_mu;
  std::string err;
  moe_status err_status = MOE_OK;
  auto record = [&](moe_status s, const std::string& m) {
    std::lock_guard<std::mutex> g(err_mu);
    if (err_status == MOE_OK) {
      err_status = s;
      err = m;
    }
    failed = true;
  };
  auto work = [&](int t) {
    bool used[2] = {false, false};
    for (int j = 0; !failed; j++) {
      const size_t i = next.fetch_add(1);
      if (i >= pieces.size()) break;
      const Piece& pc = pieces[i];
      const int slot = 2 * t + (j & 1);
      hipError_t he;
      if (used[j & 1] && (he = hipEventSynchronize(S.ev[slot])) != hipSuccess) {
        record(MOE_ERR_HIP, std::string("staging wait: ") + hipGetErrorString(he));
        break;
      }
      unsigned char* b = static_cast<unsigned char*>(S.buf[slot]);
      size_t got = 0;
      while (got < pc.n) {
        const ssize_t r = pread(pc.fd, b + got, pc.n - got, (off_t)(pc.off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
          record(MOE_ERR_INVALID, r < 0 ? std::string("read failed: ") + strerror(errno)
                                        : std::string("file shorter than its header says"));
          break;
        }
        got += (size_t)r;
      }
      if (got < pc.n) break;
      if ((he = hipMemcpyAsync(pc.dst, b, pc.n, hipMemcpyHostToDevice, st)) != hipSuccess ||
          (he = hipEventRecord(S.ev[slot], st)) != hipSuccess) {
        record(MOE_ERR_HIP, std::string("host-to-device copy: ") + hipGetErrorString(he));
        break;
      }
      used[j & 1] = true;
    }
    for (int k = 0; k < 2; k++) {
      hipError_t he;
      if (used[k] && (he = hipEventSynchronize(S.ev[2 * t + k])) != hipSuccess)
        record(MOE_ERR_HIP, std::string("staging wait: ") + hipGetErrorString(he));
    }
  };
  std::vector<std::thread> pool;
  pool.reserve((size_t)P - 1);
  for (int t = 1; t < P; t++) pool.emplace_back(work, t);
  work(0);
  for (auto& th : pool) th.join();
  if (err_status != MOE_OK) return st_fail(err_status, "upload: %s", err.c_str());
  return MOE_OK;
}

Range entry_range(const moe_st_bundle* b, const Entry& e, void* dst) {
  return Range{b->files[e.file].fd, e.offset, e.nbytes, static_cast<unsigned char*>(dst)};
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// The shapes of a stacked triplet and the bit width they imply
// (deriveAffineQuantBits, Layers.swift:348-363).
struct Stacked {
  const Entry* w;
  const Entry* s;
  const Entry* bi;
  int64_t E, N, P, G;
  int bits, sb_dtype;
  size_t w_off, s_off, b_off, total;
};

moe_status stacked_layout(const moe_st_bundle* b, const char* base, int group_size, Stacked* out) {
  if (!b || !base) return st_fail(MOE_ERR_INVALID, "load_stacked: NULL argument");
  if (group_size <= 0) return st_fail(MOE_ERR_INVALID, "load_stacked: group_size must be positive");
  const std::string nb = base;
  const std::string wn = nb + ".weight", sn = nb + ".scales", bn = nb + ".biases";
  Stacked L{};
  L.w = find(b, wn.c_str());
  L.s = find(b, sn.c_str());
  L.bi = find(b, bn.c_str());
  if (!L.w) return missing(wn.c_str());
  if (!L.s) return missing(sn.c_str());
  if (!L.bi) return missing(bn.c_str());
  const Entry& w = *L.w;
  const Entry& s = *L.s;
  const Entry& bi = *L.bi;
  if (w.dtype != MOE_ST_U32 && w.dtype != MOE_ST_I32)
    return st_fail(MOE_ERR_INVALID, "%s: packed weight must be U32 (or I32)", wn.c_str());
  if (s.dtype != MOE_ST_F32 && s.dtype != MOE_ST_F16 && s.dtype != MOE_ST_BF16)
    return st_fail(MOE_ERR_UNSUPPORTED, "%s: scales must be F32, F16 or BF16", sn.c_str());
  if (bi.dtype != s.dtype || bi.shape != s.shape)
    return st_fail(MOE_ERR_INVALID, "%s: biases must match the scales in dtype and shape",
                   bn.c_str());
  const size_t nd = w.shape.size();
  if ((nd != 2 && nd != 3) || s.shape.size() != nd)
    return st_fail(MOE_ERR_INVALID, "%s: expected [E, N, packed] or [N, packed] tensors",
                   nb.c_str());
  L.E = nd == 3 ? w.shape[0] : 1;
  L.N = w.shape[nd - 2];
  L.P = w.shape[nd - 1];
  L.G = s.shape[nd - 1];
  if ((nd == 3 && s.shape[0] != L.E) || s.shape[nd - 2] != L.N)
    return st_fail(MOE_ERR_INVALID, "%s: scales [%lld, %lld] do not match weight rows", nb.c_str(),
                   (long long)(nd == 3 ? s.shape[0] : 1), (long long)s.shape[nd - 2]);
  const int64_t K = L.G * (int64_t)group_size;
  if (L.E <= 0 || L.N <= 0 || L.P <= 0 || K <= 0)
    return st_fail(MOE_ERR_INVALID, "%s: empty stacked tensor", nb.c_str());
  if ((32 * L.P) % K != 0)
    return st_fail(MOE_ERR_INVALID,
                   "deriveAffineQuantBits: %lld packed weight columns are inconsistent with %lld "
                   "in-features at group size %d",
                   (long long)L.P, (long long)K, group_size);
  L.bits = (int)((32 * L.P) / K);
  if (L.bits != 2 && L.bits != 3 && L.bits != 4 && L.bits != 5 && L.bits != 6 && L.bits != 8)
    return st_fail(MOE_ERR_UNSUPPORTED,
                   "%s: derived %d-bit weights, an unsupported quantization bit-width", nb.c_str(),
                   L.bits);
  if (L.E > INT_MAX || L.N > INT_MAX || K > INT_MAX)
    return st_fail(MOE_ERR_UNSUPPORTED, "%s: dimensions above 2^31", nb.c_str());
  L.sb_dtype = s.dtype;
  L.w_off = 0;
  L.s_off = align256(w.nbytes);
  L.b_off = L.s_off + align256(s.nbytes);
  L.total = L.b_off + align256(bi.nbytes);
  *out = L;
  return MOE_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------

extern "C" moe_status moe_st_open(const char* path, moe_st_t* out) {
  if (!path || !out) return st_fail(MOE_ERR_INVALID, "moe_st_open: NULL argument");
  *out = nullptr;
  std::unique_ptr<moe_st_bundle> b(new (std::nothrow) moe_st_bundle());
  if (!b) return st_fail(MOE_ERR_INVALID, "moe_st_open: out of host memory");
  std::string p(path);
  while (p.size() > 1 && p.back() == '/') p.pop_back();
  if (!exists(p)) return st_fail(MOE_ERR_INVALID, "safetensors file not found: %s", p.c_str());
  std::vector<std::string> files;
  if (is_dir(p)) {
    ST_TRY(bundle_files(p, &files));
    if (files.empty())
      return st_fail(MOE_ERR_INVALID, "no .safetensors files in %s", p.c_str());
  } else {
    files.push_back(p);
  }
  for (const auto& f : files) ST_TRY(map_file(b.get(), f));
  b->names.reserve(b->entries.size());
  for (const auto& kv : b->entries) b->names.push_back(kv.first);
  std::sort(b->names.begin(), b->names.end());
  *out = b.release();
  return st_ok();
}

extern "C" void moe_st_close(moe_st_t bundle) { delete bundle; }

extern "C" int64_t moe_st_count(moe_st_t bundle) {
  return bundle ? (int64_t)bundle->names.size() : 0;
}

extern "C" const char* moe_st_name(moe_st_t bundle, int64_t i) {
  if (!bundle || i < 0 || i >= (int64_t)bundle->names.size()) return nullptr;
  return bundle->names[(size_t)i].c_str();
}

extern "C" moe_status moe_st_info(moe_st_t bundle, const char* name, int32_t* dtype,
                                  int32_t* ndim, int64_t* shape, size_t* nbytes) {
  const Entry* e = find(bundle, name);
  if (!e) return missing(name);
  if (dtype) *dtype = e->dtype;
  if (ndim) *ndim = (int32_t)e->shape.size();
  if (shape)
    for (size_t i = 0; i < e->shape.size(); i++) shape[i] = e->shape[i];
  if (nbytes) *nbytes = e->nbytes;
  return st_ok();
}

extern "C" moe_status moe_st_read_host(moe_st_t bundle, const char* name, void* dst,
                                       size_t bytes) {
  const Entry* e = find(bundle, name);
  if (!e) return missing(name);
  if (!dst && e->nbytes) return st_fail(MOE_ERR_INVALID, "read_host: NULL destination");
  if (bytes != e->nbytes)
    return st_fail(MOE_ERR_INVALID, "read_host: tensor \"%s\" holds %zu bytes, not %zu", name,
                   e->nbytes, bytes);
  if (bytes) memcpy(dst, entry_bytes(bundle, *e), bytes);
  return st_ok();
}

extern "C" moe_status moe_st_upload(moe_st_t bundle, const char* name, void* dst_device,
                                    size_t bytes, hipStream_t stream) {
  const Entry* e = find(bundle, name);
  if (!e) return missing(name);
  if (!dst_device && e->nbytes) return st_fail(MOE_ERR_INVALID, "upload: NULL destination");
  if (bytes != e->nbytes)
    return st_fail(MOE_ERR_INVALID, "upload: tensor \"%s\" holds %zu bytes, not %zu", name,
                   e->nbytes, bytes);
  ST_TRY(upload_ranges({entry_range(bundle, *e, dst_device)}, stream));
  return st_ok();
}

extern "C" int32_t moe_st_is_quantized(moe_st_t bundle, const char* base) {
  if (!bundle || !base) return 0;
  const std::string nb = base;
  return find(bundle, (nb + ".weight").c_str()) && find(bundle, (nb + ".scales").c_str()) &&
         find(bundle, (nb + ".biases").c_str());
}

extern "C" moe_status moe_st_stacked_bytes(moe_st_t bundle, const char* base, int32_t group_size,
                                           size_t* bytes) {
  if (!bytes) return st_fail(MOE_ERR_INVALID, "stacked_bytes: NULL argument");
  Stacked L;
  ST_TRY(stacked_layout(bundle, base, group_size, &L));
  *bytes = L.total;
  return st_ok();
}

namespace {

// Validates one triplet against its destination and appends its three ranges.
moe_status plan_stacked(const moe_st_bundle* b, const char* base, int group_size, void* dst,
                        size_t dst_bytes, moe_qproj* q, std::vector<Range>* ranges) {
  Stacked L;
  ST_TRY(stacked_layout(b, base, group_size, &L));
  if (!dst || dst_bytes < L.total)
    return st_fail(MOE_ERR_INVALID, "load_stacked: %s needs %zu device bytes", base, L.total);
  if ((reinterpret_cast<uintptr_t>(dst) & 255) != 0)
    return st_fail(MOE_ERR_INVALID, "load_stacked: destination must be 256-byte aligned");
  unsigned char* d = static_cast<unsigned char*>(dst);
  *q = moe_qproj{};
  q->weight = reinterpret_cast<const uint32_t*>(d + L.w_off);
  q->scales = d + L.s_off;
  q->biases = d + L.b_off;
  q->out_bias = nullptr;
  q->bits = L.bits;
  q->group_size = group_size;
  q->sb_dtype = L.sb_dtype;
  q->n = (int32_t)L.N;
  q->k = (int32_t)(L.G * group_size);
  q->n_experts = (int32_t)L.E;
  // the kernels' own contract (bit width, group size, alignment) before any copy
  ST_TRY(moe_validate_qproj(q));
  ranges->push_back(entry_range(b, *L.w, d + L.w_off));
  ranges->push_back(entry_range(b, *L.s, d + L.s_off));
  ranges->push_back(entry_range(b, *L.bi, d + L.b_off));
  return MOE_OK;
}

}  // namespace

extern "C" moe_status moe_st_load_stacked(moe_st_t bundle, const char* base, int32_t group_size,
                                          void* dst_device, size_t dst_bytes, moe_qproj* out,
                                          hipStream_t stream) {
  return moe_st_load_stacked_many(bundle, 1, &base, group_size, &dst_device, &dst_bytes, out,
                                  stream);
}

extern "C" moe_status moe_st_load_stacked_many(moe_st_t bundle, int32_t count,
                                               const char* const* bases, int32_t group_size,
                                               void* const* dst_device, const size_t* dst_bytes,
                                               moe_qproj* out, hipStream_t stream) {
  if (count <= 0 || !bases || !dst_device || !dst_bytes || !out)
    return st_fail(MOE_ERR_INVALID, "load_stacked: NULL argument or empty list");
  std::vector<Range> ranges;
  std::vector<moe_qproj> qs((size_t)count);
  for (int i = 0; i < count; i++)
    ST_TRY(plan_stacked(bundle, bases[i], group_size, dst_device[i], dst_bytes[i], &qs[(size_t)i],
                        &ranges));
  ST_TRY(upload_ranges(ranges, stream));
  for (int i = 0; i < count; i++) out[i] = qs[(size_t)i];
  return st_ok();
}

// ---------------------------------------------------------------------------
// MXFP4 expert stacks (GPT-OSS)
// ---------------------------------------------------------------------------
namespace {

// <base>.weight [E, N, K/8] u32, <base>.scales [E, N, K/32] u8 (e8m0),
// <base>.bias [E, N] f16/bf16/f32 (transcodeStackedExperts,
// GPTOSSText.swift:1071-1110); 2-D tensors are one expert.
struct Mxfp4 {
  const Entry* w;
  const Entry* s;
  const Entry* bi;
  int64_t E, N, G;
  size_t w_off, s_off, b_off, ob_off, total;   // device layout
  size_t sc_e8m0, sc_bias, scratch;            // scratch layout
};

moe_status mxfp4_layout(const moe_st_bundle* b, const char* base, int act_dtype, Mxfp4* out) {
  if (!b || !base) return st_fail(MOE_ERR_INVALID, "load_mxfp4: NULL argument");
  if (act_dtype != MOE_ST_F32 && act_dtype != MOE_ST_F16 && act_dtype != MOE_ST_BF16)
    return st_fail(MOE_ERR_INVALID, "load_mxfp4: bad activation dtype %d", act_dtype);
  const std::string nb = base;
  const std::string wn = nb + ".weight", sn = nb + ".scales", bn = nb + ".bias";
  Mxfp4 L{};
  L.w = find(b, wn.c_str());
  L.s = find(b, sn.c_str());
  L.bi = find(b, bn.c_str());
  if (!L.w) return missing(wn.c_str());
  if (!L.s) return missing(sn.c_str());
  if (!L.bi) return missing(bn.c_str());
  if (L.w->dtype != MOE_ST_U32)
    return st_fail(MOE_ERR_INVALID, "GPT-OSS MoE: %s expected u32", wn.c_str());
  if (L.s->dtype != MOE_ST_U8)
    return st_fail(MOE_ERR_INVALID, "GPT-OSS MoE: %s expected u8", sn.c_str());
  if (L.bi->dtype != MOE_ST_F32 && L.bi->dtype != MOE_ST_F16 && L.bi->dtype != MOE_ST_BF16)
    return st_fail(MOE_ERR_INVALID, "GPT-OSS MoE: %s must be f16, bf16 or f32", bn.c_str());
  const size_t nd = L.w->shape.size();
  if ((nd != 2 && nd != 3) || L.s->shape.size() != nd || L.bi->shape.size() != nd - 1)
    return st_fail(MOE_ERR_INVALID, "GPT-OSS MoE: %s expected [E, N, K/8] / [E, N, K/32] / [E, N]",
                   nb.c_str());
  L.E = nd == 3 ? L.w->shape[0] : 1;
  L.N = L.w->shape[nd - 2];
  L.G = L.s->shape[nd - 1];
  const int64_t words = L.w->shape[nd - 1];
  if ((nd == 3 && (L.s->shape[0] != L.E || L.bi->shape[0] != L.E)) || L.s->shape[nd - 2] != L.N ||
      L.bi->shape[nd - 2] != L.N || words != 4 * L.G || L.E <= 0 || L.N <= 0 || L.G <= 0)
    return st_fail(MOE_ERR_INVALID,
                   "GPT-OSS MoE: %s weight, scales and bias shapes disagree (32 codes per scale)",
                   nb.c_str());
  if (L.E > INT_MAX || L.N > INT_MAX || 32 * L.G > INT_MAX)
    return st_fail(MOE_ERR_UNSUPPORTED, "%s: dimensions above 2^31", nb.c_str());
  const size_t ds = act_dtype == MOE_ST_F32 ? 4 : 2;
  const size_t groups = (size_t)(L.E * L.N * L.G);
  L.w_off = 0;
  L.s_off = align256(L.w->nbytes);
  L.b_off = L.s_off + align256(groups * ds);
  L.ob_off = L.b_off + align256(groups * ds);
  L.total = L.ob_off + align256((size_t)(L.E * L.N) * ds);
  L.sc_e8m0 = 0;
  L.sc_bias = align256(L.s->nbytes);
  L.scratch = L.sc_bias + align256(L.bi->nbytes);
  *out = L;
  return MOE_OK;
}

}  // namespace

extern "C" moe_status moe_st_mxfp4_bytes(moe_st_t bundle, const char* base, int32_t act_dtype,
                                         size_t* bytes, size_t* scratch_bytes) {
  if (!bytes || !scratch_bytes) return st_fail(MOE_ERR_INVALID, "mxfp4_bytes: NULL argument");
  Mxfp4 L;
  ST_TRY(mxfp4_layout(bundle, base, act_dtype, &L));
  *bytes = L.total;
  *scratch_bytes = L.scratch;
  return st_ok();
}

extern "C" moe_status moe_st_load_mxfp4(moe_st_t bundle, const char* base, int32_t act_dtype,
                                        void* dst_device, size_t dst_bytes, void* scratch_device,
                                        size_t scratch_bytes, moe_qproj* out,
                                        hipStream_t stream) {
  if (!out) return st_fail(MOE_ERR_INVALID, "load_mxfp4: NULL output descriptor");
  Mxfp4 L;
  ST_TRY(mxfp4_layout(bundle, base, act_dtype, &L));
  if (!dst_device || dst_bytes < L.total)
    return st_fail(MOE_ERR_INVALID, "load_mxfp4: %s needs %zu device bytes", base, L.total);
  if (!scratch_device || scratch_bytes < L.scratch)
    return st_fail(MOE_ERR_INVALID, "load_mxfp4: %s needs %zu scratch bytes", base, L.scratch);
  if ((reinterpret_cast<uintptr_t>(dst_device) & 255) ||
      (reinterpret_cast<uintptr_t>(scratch_device) & 255))
    return st_fail(MOE_ERR_INVALID, "load_mxfp4: buffers must be 256-byte aligned");
  unsigned char* d = static_cast<unsigned char*>(dst_device);
  unsigned char* sc = static_cast<unsigned char*>(scratch_device);
  moe_qproj q{};
  q.weight = reinterpret_cast<const uint32_t*>(d + L.w_off);
  q.scales = d + L.s_off;
  q.biases = d + L.b_off;
  q.out_bias = d + L.ob_off;
  q.bits = 4;
  q.group_size = 32;
  q.sb_dtype = act_dtype;
  q.n = (int32_t)L.N;
  q.k = (int32_t)(32 * L.G);
  q.n_experts = (int32_t)L.E;
  ST_TRY(moe_validate_qproj(&q));
  ST_TRY(upload_ranges({entry_range(bundle, *L.w, d + L.w_off),
                        entry_range(bundle, *L.s, sc + L.sc_e8m0),
                        entry_range(bundle, *L.bi, sc + L.sc_bias)},
                       stream));
  // the codes transcode in place; scales and biases land in act_dtype
  hipError_t e = moe::launch_mxfp4_affine(reinterpret_cast<const uint32_t*>(d + L.w_off),
                                          sc + L.sc_e8m0, L.E * L.N * L.G,
                                          reinterpret_cast<uint32_t*>(d + L.w_off), d + L.s_off,
                                          d + L.b_off, act_dtype, stream);
  if (e == hipSuccess)
    e = moe::launch_convert(sc + L.sc_bias, L.bi->dtype, d + L.ob_off, act_dtype, L.E * L.N,
                            stream);
  if (e != hipSuccess) return hip_fail(e, "MXFP4 transcode launch");
  *out = q;
  return st_ok();
}

