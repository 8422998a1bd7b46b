// blob.cpp -- the .lfm3q8 weight blob: header parser, crc32-checked tensor
// reads, and the reader that pipelines file reads with the caller's work.
//
// Format (written by export_lfm3_q8.py:37-41, 172-180; read by load_blob,
// lfm3_nanode.cu:1219-1733):
//   8 bytes magic "LFM3Q8\x01\x00"; uint32 little-endian header length n;
//   n bytes of JSON {"magic", "cfg", "n_tensors", "vocab_size", "hidden_size",
//   "data_bytes", "table": [{"name", "dtype", "ne", "off", "ncodes", "nscales",
//   "crc"}, ...]}; then the payloads, tensor i at (12 + n) + off_i: ncodes
//   bytes (int8 codes for dtype 1, f32 for 2, bf16 for 3) followed by nscales
//   bytes of fp32 scales (one per 32 codes, dtype 1 only); dtype 6 / 7 are the
//   Q4 / Q5 tensors .auto/lfm3/export_qlow.py writes, pre-tiled in 32-row tiles
//   (16 / 20 code bytes per 32-group, then 4 bytes of (d', mn) fp16). crc is the zlib
//   crc32 of the payload (codes then scales), recomputed here on the bytes
//   read, as the reference's loader does (1358-1362).
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <condition_variable>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "../../include/pulsar_amd.h"
#include "pq_host.h"
#include "pq_internal.h"

namespace pq {

// ------------------------------------------------------------------- crc32
// The zlib / IEEE 802.3 CRC-32 (reflected polynomial 0xEDB88320, initial and
// final complement), eight table lookups per 8 bytes.
static uint32_t g_crc_tab[8][256];
static std::once_flag g_crc_once;
static void crc_init() {
  for (uint32_t i = 0; i < 256; i++) {
    uint32_t c = i;
    for (int k = 0; k < 8; k++) c = (c & 1) ? 0xEDB88320u ^ (c >> 1) : c >> 1;
    g_crc_tab[0][i] = c;
  }
  for (uint32_t i = 0; i < 256; i++)
    for (int t = 1; t < 8; t++) g_crc_tab[t][i] = (g_crc_tab[t - 1][i] >> 8) ^ g_crc_tab[0][g_crc_tab[t - 1][i] & 0xff];
}
uint32_t crc32_update(uint32_t crc, const void *data, size_t n) {
  std::call_once(g_crc_once, crc_init);
  const uint8_t *p = static_cast<const uint8_t *>(data);
  uint32_t c = ~crc;
  while (n >= 8) {
    uint32_t lo, hi;
    memcpy(&lo, p, 4);
    memcpy(&hi, p + 4, 4);
    lo ^= c;
    c = g_crc_tab[7][lo & 0xff] ^ g_crc_tab[6][(lo >> 8) & 0xff] ^ g_crc_tab[5][(lo >> 16) & 0xff] ^
        g_crc_tab[4][lo >> 24] ^ g_crc_tab[3][hi & 0xff] ^ g_crc_tab[2][(hi >> 8) & 0xff] ^
        g_crc_tab[1][(hi >> 16) & 0xff] ^ g_crc_tab[0][hi >> 24];
    p += 8;
    n -= 8;
  }
  while (n--) c = g_crc_tab[0][(c ^ *p++) & 0xff] ^ (c >> 8);
  return ~c;
}

// -------------------------------------------------------------------- JSON
// Enough of JSON for the header: objects, arrays, strings (with \" \\ \/
// \n \t \r \b \f \uXXXX below 0x80), numbers, true / false / null.
struct Json {
  enum Kind { Null, Bool, Num, Str, Arr, Obj } kind = Null;
  double num = 0;
  bool b = false;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json *get(const char *k) const {
    for (const auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char *p, *end;
  std::string err;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\n' || *p == '\t' || *p == '\r')) p++;
  }
  bool fail(const char *m) {
    if (err.empty()) err = m;
    return false;
  }
  bool str(std::string &out) {
    if (p >= end || *p != '"') return fail("expected a string");
    p++;
    while (p < end && *p != '"') {
      char ch = *p++;
      if (ch == '\\') {
        if (p >= end) return fail("bad escape");
        const char e = *p++;
        switch (e) {
          case '"': ch = '"'; break;
          case '\\': ch = '\\'; break;
          case '/': ch = '/'; break;
          case 'n': ch = '\n'; break;
          case 't': ch = '\t'; break;
          case 'r': ch = '\r'; break;
          case 'b': ch = '\b'; break;
          case 'f': ch = '\f'; break;
          case 'u': {
            if (end - p < 4) return fail("bad \\u escape");
            const std::string hex(p, p + 4);
            p += 4;
            const long v = strtol(hex.c_str(), nullptr, 16);
            if (v >= 0x80) return fail("non-ASCII \\u escape");
            ch = (char)v;
            break;
          }
          default: return fail("bad escape");
        }
      }
      out.push_back(ch);
    }
    if (p >= end) return fail("unterminated string");
    p++;
    return true;
  }
  bool value(Json &v, int depth) {
    if (depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    if (*p == '{') {
      v.kind = Json::Obj;
      p++;
      ws();
      if (p < end && *p == '}') { p++; return true; }
      for (;;) {
        ws();
        std::string k;
        if (!str(k)) return false;
        ws();
        if (p >= end || *p != ':') return fail("expected ':'");
        p++;
        v.obj.emplace_back(std::move(k), Json());
        if (!value(v.obj.back().second, depth + 1)) return false;
        ws();
        if (p < end && *p == ',') { p++; continue; }
        if (p < end && *p == '}') { p++; return true; }
        return fail("expected ',' or '}'");
      }
    }
    if (*p == '[') {
      v.kind = Json::Arr;
      p++;
      ws();
      if (p < end && *p == ']') { p++; return true; }
      for (;;) {
        v.arr.emplace_back();
        if (!value(v.arr.back(), depth + 1)) return false;
        ws();
        if (p < end && *p == ',') { p++; continue; }
        if (p < end && *p == ']') { p++; return true; }
        return fail("expected ',' or ']'");
      }
    }
    if (*p == '"') { v.kind = Json::Str; return str(v.str); }
    if (end - p >= 4 && !strncmp(p, "true", 4)) { v.kind = Json::Bool; v.b = true; p += 4; return true; }
    if (end - p >= 5 && !strncmp(p, "false", 5)) { v.kind = Json::Bool; p += 5; return true; }
    if (end - p >= 4 && !strncmp(p, "null", 4)) { p += 4; return true; }
    const char *q = p;
    while (q < end && (strchr("+-0123456789.eE", *q) != nullptr)) q++;
    if (q == p) return fail("unexpected character");
    const std::string num(p, q);
    char *ep = nullptr;
    v.num = strtod(num.c_str(), &ep);
    if (ep != num.c_str() + num.size()) return fail("bad number");
    v.kind = Json::Num;
    p = q;
    return true;
  }
};

static void json_write(const Json &v, std::string &o) {
  char buf[64];
  switch (v.kind) {
    case Json::Null: o += "null"; break;
    case Json::Bool: o += v.b ? "true" : "false"; break;
    case Json::Num:
      if (v.num == (double)(long long)v.num && v.num < 9e15 && v.num > -9e15) snprintf(buf, sizeof buf, "%lld", (long long)v.num);
      else snprintf(buf, sizeof buf, "%.17g", v.num);
      o += buf;
      break;
    case Json::Str:
      o += '"';
      for (char ch : v.str) {
        if (ch == '"' || ch == '\\') { o += '\\'; o += ch; }
        else if ((unsigned char)ch < 0x20) { snprintf(buf, sizeof buf, "\\u%04x", ch); o += buf; }
        else o += ch;
      }
      o += '"';
      break;
    case Json::Arr:
      o += '[';
      for (size_t i = 0; i < v.arr.size(); i++) {
        if (i) o += ',';
        json_write(v.arr[i], o);
      }
      o += ']';
      break;
    case Json::Obj:
      o += '{';
      for (size_t i = 0; i < v.obj.size(); i++) {
        if (i) o += ',';
        Json k;
        k.kind = Json::Str;
        k.str = v.obj[i].first;
        json_write(k, o);
        o += ':';
        json_write(v.obj[i].second, o);
      }
      o += '}';
      break;
  }
}

// -------------------------------------------------------------------- blob
struct BlobEnt {
  std::string name;
  int dtype = 0, ndim = 0;
  long long ne[4] = {0, 0, 0, 0};
  uint64_t off = 0, ncodes = 0, nscales = 0;
  uint32_t crc = 0;
};

struct Blob {
  int fd = -1;
  uint64_t base = 0, fsize = 0;
  std::vector<BlobEnt> ents;
  std::map<std::string, int> index;
  std::string cfg;
  ~Blob() {
    if (fd >= 0) close(fd);
  }
};

static const char kMagic[8] = {'L', 'F', 'M', '3', 'Q', '8', 1, 0};
constexpr size_t kReadPiece = (size_t)16 << 20;   // pread size, as the reference's ring (1221)

static bool get_u64(const Json &o, const char *k, uint64_t &out) {
  const Json *v = o.get(k);
  if (!v || v->kind != Json::Num || v->num < 0 || v->num > 1.8e19) return false;
  out = (uint64_t)v->num;
  return (double)out == v->num;
}

static Blob *blob_open(const char *path) {
  std::unique_ptr<Blob> B(new Blob);
  B->fd = open(path, O_RDONLY);
  if (B->fd < 0) { fail(PQ_ERR_ARG, "blob: cannot open %s", path); return nullptr; }
  struct stat st;
  if (fstat(B->fd, &st) != 0) { fail(PQ_ERR_ARG, "blob: cannot stat %s", path); return nullptr; }
  B->fsize = (uint64_t)st.st_size;
  char head[12];
  if (B->fsize < 12 || pread(B->fd, head, 12, 0) != 12 || memcmp(head, kMagic, 8) != 0) {
    fail(PQ_ERR_ARG, "blob: %s is not an .lfm3q8 file (magic)", path);
    return nullptr;
  }
  uint32_t n;
  memcpy(&n, head + 8, 4);
  if ((uint64_t)n + 12 > B->fsize) { fail(PQ_ERR_ARG, "blob: header length %u past the end of the file", n); return nullptr; }
  std::string hj(n, '\0');
  if (pread(B->fd, &hj[0], n, 12) != (ssize_t)n) { fail(PQ_ERR_ARG, "blob: short header read"); return nullptr; }
  B->base = 12 + (uint64_t)n;
  Json h;
  JsonParser jp{hj.data(), hj.data() + hj.size(), {}};
  if (!jp.value(h, 0) || h.kind != Json::Obj) {
    fail(PQ_ERR_ARG, "blob: header is not a JSON object (%s)", jp.err.c_str());
    return nullptr;
  }
  const Json *tab = h.get("table");
  if (!tab || tab->kind != Json::Arr) { fail(PQ_ERR_ARG, "blob: header has no tensor table"); return nullptr; }
  uint64_t data_bytes = 0;
  if (h.get("data_bytes") && !get_u64(h, "data_bytes", data_bytes)) {
    fail(PQ_ERR_ARG, "blob: bad data_bytes");
    return nullptr;
  }
  for (const Json &t : tab->arr) {
    BlobEnt e;
    const Json *nm = t.get("name"), *dt = t.get("dtype"), *ne = t.get("ne");
    uint64_t crc = 0;
    if (t.kind != Json::Obj || !nm || nm->kind != Json::Str || !dt || dt->kind != Json::Num || !ne ||
        ne->kind != Json::Arr || ne->arr.empty() || ne->arr.size() > 4 || !get_u64(t, "off", e.off) ||
        !get_u64(t, "ncodes", e.ncodes) || !get_u64(t, "nscales", e.nscales) || !get_u64(t, "crc", crc) ||
        crc > 0xffffffffull) {
      fail(PQ_ERR_ARG, "blob: malformed table entry %zu", B->ents.size());
      return nullptr;
    }
    e.name = nm->str;
    e.dtype = (int)dt->num;
    e.crc = (uint32_t)crc;
    e.ndim = (int)ne->arr.size();
    // every size is bounded by the file's: an element count past 2 * fsize (Q4
    // stores 0.625 bytes per element; or a product that would overflow on the
    // way there) cannot be a real tensor
    uint64_t elems = 1;
    for (int d = 0; d < e.ndim; d++) {
      if (ne->arr[d].kind != Json::Num || ne->arr[d].num < 1 || ne->arr[d].num > 1e12) {
        fail(PQ_ERR_ARG, "blob: %s has a bad shape", e.name.c_str());
        return nullptr;
      }
      e.ne[d] = (long long)ne->arr[d].num;
      if (__builtin_mul_overflow(elems, (uint64_t)e.ne[d], &elems) || elems > 2 * (uint64_t)B->fsize) {
        fail(PQ_ERR_ARG, "blob: %s has more elements than the file can hold", e.name.c_str());
        return nullptr;
      }
    }
    // the payload must be what the shape and dtype say (export_lfm3_q8.py:132-155)
    bool ok = false;
    if (e.dtype == 1) ok = e.ndim == 2 && e.ne[1] % 32 == 0 && e.ncodes == elems && e.nscales == elems / 8;
    else if (e.dtype == 2) ok = e.ncodes == elems * 4 && e.nscales == 0;      // elems <= 2 fsize: no overflow
    else if (e.dtype == 3) ok = e.ncodes == elems * 2 && e.nscales == 0;
    else if (e.dtype == 6 || e.dtype == 7)   // Q4 / Q5, pre-tiled (lfm3_nanode.cu:1494-1500)
      ok = e.ndim == 2 && e.ne[0] % 32 == 0 && e.ne[1] % 256 == 0 &&
           e.ncodes == elems / 32 * (e.dtype == 6 ? 16 : 20) && e.nscales == elems / 32 * 4;
    if (!ok) {
      fail(PQ_ERR_ARG, "blob: %s: dtype %d with %llu + %llu payload bytes does not match its shape", e.name.c_str(),
           e.dtype, (unsigned long long)e.ncodes, (unsigned long long)e.nscales);
      return nullptr;
    }
    // each term is checked against fsize before the sum, so it cannot wrap
    if (e.off > B->fsize || e.ncodes > B->fsize || e.nscales > B->fsize ||
        B->base + e.off + e.ncodes + e.nscales > B->fsize) {
      fail(PQ_ERR_ARG, "blob: %s extends past the end of the file (truncated?)", e.name.c_str());
      return nullptr;
    }
    if (B->index.count(e.name)) { fail(PQ_ERR_ARG, "blob: tensor %s listed twice", e.name.c_str()); return nullptr; }
    B->index[e.name] = (int)B->ents.size();
    B->ents.push_back(std::move(e));
  }
  if (const Json *cfg = h.get("cfg")) json_write(*cfg, B->cfg);
  else B->cfg = "{}";
  return B.release();
}

// Tensor i's payload into dst0 (codes) and dst1 (scales), crc checked.
static int blob_read(Blob &B, int i, void *dst0, void *dst1) {
  PQ_REQUIRE(i >= 0 && i < (int)B.ents.size(), PQ_ERR_ARG, "blob: no tensor %d", i);
  const BlobEnt &e = B.ents[i];
  PQ_REQUIRE(dst0 && (e.nscales == 0 || dst1), PQ_ERR_ARG, "blob: %s: null destination", e.name.c_str());
  uint32_t c = 0;
  const uint64_t tot = e.ncodes + e.nscales;
  for (uint64_t done = 0; done < tot;) {
    const bool codes = done < e.ncodes;
    const uint64_t lim = codes ? e.ncodes : tot;
    const size_t n = (size_t)std::min<uint64_t>(lim - done, kReadPiece);
    char *dst = codes ? static_cast<char *>(dst0) + done : static_cast<char *>(dst1) + (done - e.ncodes);
    size_t got = 0;
    while (got < n) {
      const ssize_t r = pread(B.fd, dst + got, n - got, (off_t)(B.base + e.off + done + got));
      if (r <= 0) return fail(PQ_ERR_ARG, "blob: short read of %s", e.name.c_str());
      got += (size_t)r;
    }
    c = crc32_update(c, dst, n);
    done += n;
  }
  PQ_REQUIRE(c == e.crc, PQ_ERR_DATA, "blob: crc mismatch in %s: read %08x, table %08x", e.name.c_str(), c, e.crc);
  return PQ_OK;
}

// ------------------------------------------------- reader for the engine load
// A thread reads the tensors in the order asked into host buffers (crc
// checked) while the caller converts and uploads the previous ones; at most
// `depth` read tensors wait.
struct BlobReader::Impl {
  Blob *B;
  std::vector<int> order;
  size_t depth;
  std::mutex mu;
  std::condition_variable cv;
  std::map<int, std::vector<char>> ready;   // order position -> payload
  int next_take = 0, status = PQ_OK;
  bool stop = false;
  std::thread th;
  std::string err;
  void run() {
    for (size_t k = 0; k < order.size(); k++) {
      {
        std::unique_lock<std::mutex> lk(mu);
        cv.wait(lk, [&] { return stop || ready.size() < depth; });
        if (stop) return;
      }
      const BlobEnt &e = B->ents[order[k]];
      std::vector<char> buf;
      int rc = PQ_OK;
      try {
        buf.resize(e.ncodes + e.nscales);
      } catch (...) {
        rc = fail(PQ_ERR_ARG, "blob: cannot allocate %llu bytes for %s",
                  (unsigned long long)(e.ncodes + e.nscales), e.name.c_str());
      }
      if (rc == PQ_OK) rc = blob_read(*B, order[k], buf.data(), buf.data() + e.ncodes);
      std::unique_lock<std::mutex> lk(mu);
      if (rc != PQ_OK) {
        status = rc;
        err = pq_last_error();
        cv.notify_all();
        return;
      }
      ready[(int)k] = std::move(buf);
      cv.notify_all();
    }
  }
};

BlobReader::BlobReader(void *blob, const std::vector<int> &order, size_t depth) : impl(new Impl) {
  impl->B = static_cast<Blob *>(blob);
  impl->order = order;
  impl->depth = depth < 1 ? 1 : depth;
  impl->th = std::thread([this] { impl->run(); });
}
BlobReader::~BlobReader() {
  {
    std::lock_guard<std::mutex> lk(impl->mu);
    impl->stop = true;
  }
  impl->cv.notify_all();
  impl->th.join();
}
int BlobReader::take(std::vector<char> &out) {
  std::unique_lock<std::mutex> lk(impl->mu);
  const int k = impl->next_take;
  impl->cv.wait(lk, [&] { return impl->ready.count(k) || impl->status != PQ_OK; });
  if (!impl->ready.count(k)) return fail(impl->status, "%s", impl->err.c_str());
  out = std::move(impl->ready[k]);
  impl->ready.erase(k);
  impl->next_take++;
  impl->cv.notify_all();
  return PQ_OK;
}

int blob_find(void *blob, const char *name) {
  Blob &B = *static_cast<Blob *>(blob);
  auto it = B.index.find(name);
  return it == B.index.end() ? -1 : it->second;
}

}  // namespace pq

using namespace pq;

extern "C" void *pq_blob_open(const char *path) {
  if (!path) { fail(PQ_ERR_ARG, "pq_blob_open: null path"); return nullptr; }
  return blob_open(path);
}

extern "C" int pq_blob_close(void *blob) {
  PQ_REQUIRE(blob, PQ_ERR_ARG, "pq_blob_close: null blob");
  delete static_cast<Blob *>(blob);
  return PQ_OK;
}

extern "C" int pq_blob_count(void *blob) {
  PQ_REQUIRE(blob, PQ_ERR_ARG, "pq_blob_count: null blob");
  return (int)static_cast<Blob *>(blob)->ents.size();
}

extern "C" int pq_blob_find(void *blob, const char *name) {
  PQ_REQUIRE(blob && name, PQ_ERR_ARG, "pq_blob_find: null argument");
  return blob_find(blob, name);
}

extern "C" int pq_blob_tensor_info(void *blob, int i, pq_blob_tensor *out) {
  PQ_REQUIRE(blob && out, PQ_ERR_ARG, "pq_blob_tensor_info: null argument");
  Blob &B = *static_cast<Blob *>(blob);
  PQ_REQUIRE(i >= 0 && i < (int)B.ents.size(), PQ_ERR_ARG, "pq_blob_tensor_info: no tensor %d", i);
  const BlobEnt &e = B.ents[i];
  memset(out, 0, sizeof *out);
  snprintf(out->name, sizeof out->name, "%s", e.name.c_str());
  out->dtype = e.dtype;
  out->ndim = e.ndim;
  for (int d = 0; d < 4; d++) out->ne[d] = e.ne[d];
  out->ncodes = (long long)e.ncodes;
  out->nscales = (long long)e.nscales;
  out->crc = e.crc;
  return PQ_OK;
}

extern "C" int pq_blob_read(void *blob, int i, void *codes, void *scales) {
  PQ_REQUIRE(blob, PQ_ERR_ARG, "pq_blob_read: null blob");
  return blob_read(*static_cast<Blob *>(blob), i, codes, scales);
}

extern "C" const char *pq_blob_config(void *blob) {
  if (!blob) return "";
  return static_cast<Blob *>(blob)->cfg.c_str();
}

extern "C" unsigned pq_crc32(unsigned crc, const void *data, size_t n) { return crc32_update(crc, data, n); }
