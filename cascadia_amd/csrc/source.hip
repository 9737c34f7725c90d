// source.hip -- the crate's C handle API (crates/cascadia-int4-gemm/src/c_ffi.rs:35-341):
// a safetensors model directory opened as an expert source, experts brought
// into HBM on first use, and one expert run on one f32 vector.
//
//   cascadia_int4_open_source(model_dir, &h)   c_ffi.rs:35-56
//   cascadia_int4_destroy_source(h)            c_ffi.rs:58-64
//   cascadia_int4_prewarm(h, layer, expert)    c_ffi.rs:66-106
//   cascadia_int4_expert_forward(h, layer, expert, x_f32, out_f32)
//                                              c_ffi.rs:305-341
//
// The source follows safetensors_source.rs:205-380: `model.safetensors.index.json`
// maps tensor names to shard files; a shard is an 8-byte little-endian header
// length, a JSON header {name: {dtype, shape, data_offsets}} and the data.
// Expert (L, E) is the six tensors
// `language_model.model.layers.L.mlp.experts.E.{gate,up,down}_proj.weight_{packed,scale}`
// (compressed-tensors: packed int32 [rows, cols / 8], whose little-endian
// bytes are the crate layout; scales bf16 or f16 [rows, cols / G]).
//
// A directory whose manifest.json says "experts_format": "int4_bin" is read
// as the runners' flat-expert layout instead (manifest.rs:137-142,
// ov_moe.rs:786-806): experts/layer_LL/expert_EEE.bin, each the six sections
// gate_p, gate_s, up_p, up_s, down_p, down_s of format.rs:35-47 with groups
// of 32 and bf16 scales; hidden = "hidden_size", intermediate =
// "expert_intermediate" (0 or absent: the crate's 2048, format.rs:51-126).
//
// Where the crate mmaps the files and lets the OS page an expert in and out
// (prewarm touches its pages), here an expert is read once, uploaded, tiled
// into the MFMA layout and kept in HBM, in an LRU cache modelled on the
// runner's (runner.rs:142-258): bounded by a count of experts and a byte
// budget (cascadia_int4_source_set_cache_limits, or the environment variables
// CASCADIA_INT4_MAX_CACHED_EXPERTS / CASCADIA_INT4_EXPERT_CACHE_BYTES at open;
// 0 = unbounded), the least recently used expert evicted once the handle's
// stream has drained; a device allocation that fails evicts and retries
// before it is reported.  prewarm does the load.  expert_forward converts x to bf16
// as the crate does (bf16::from_f32: RNE, NaN made quiet), runs
// cascadia_int4_expert_forward_device and widens the bf16 result to f32; it
// is synchronous, like the crate's.  The hidden size is the model's (7168 in
// the crate's HIDDEN); x and out hold that many floats.
//
// Return codes as the crate's: 0 OK, -1 null argument, -2 invalid UTF-8 path
// (open) or an expert that cannot be read (prewarm / forward), -3 a model
// directory that cannot be opened; a HIP failure returns -3 as well.
#include <fcntl.h>
#include <unistd.h>

#include <sys/stat.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <condition_variable>
#include <deque>
#include <list>
#include <set>
#include <thread>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/cascadia_int4.h"
#include "int4_common.hpp"

namespace {

// ---------------------------------------------------------------------------
// a small JSON reader (objects, arrays, strings, numbers, literals): enough
// for the index file and safetensors headers
// ---------------------------------------------------------------------------

struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  double num = 0;
  std::string str;
  std::vector<Json> arr;
  std::vector<std::pair<std::string, Json>> obj;
  const Json *get(const std::string &k) const {
    for (const auto &kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct JsonParser {
  const char *p, *end;
  bool ok = true;
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool lit(const char *s) {
    const size_t n = strlen(s);
    if ((size_t)(end - p) < n || strncmp(p, s, n) != 0) return false;
    p += n;
    return true;
  }
  static void utf8(std::string &out, unsigned c) {
    if (c < 0x80) {
      out += (char)c;
    } else if (c < 0x800) {
      out += (char)(0xC0 | (c >> 6));
      out += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      out += (char)(0xE0 | (c >> 12));
      out += (char)(0x80 | ((c >> 6) & 0x3F));
      out += (char)(0x80 | (c & 0x3F));
    } else {
      out += (char)(0xF0 | (c >> 18));
      out += (char)(0x80 | ((c >> 12) & 0x3F));
      out += (char)(0x80 | ((c >> 6) & 0x3F));
      out += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(unsigned &v) {
    if (end - p < 4) return false;
    v = 0;
    for (int i = 0; i < 4; ++i) {
      const char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
      else return false;
    }
    return true;
  }
  bool string(std::string &out) {
    if (p >= end || *p != '"') return false;
    ++p;
    while (p < end && *p != '"') {
      if (*p == '\\') {
        if (++p >= end) return false;
        const char e = *p++;
        switch (e) {
          case '"': out += '"'; break;
          case '\\': out += '\\'; break;
          case '/': out += '/'; break;
          case 'b': out += '\b'; break;
          case 'f': out += '\f'; break;
          case 'n': out += '\n'; break;
          case 'r': out += '\r'; break;
          case 't': out += '\t'; break;
          case 'u': {
            unsigned c;
            if (!hex4(c)) return false;
            if (c >= 0xD800 && c < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
              p += 2;
              unsigned lo;
              if (!hex4(lo)) return false;
              c = 0x10000 + ((c - 0xD800) << 10) + (lo - 0xDC00);
            }
            utf8(out, c);
            break;
          }
          default: return false;
        }
      } else {
        out += *p++;
      }
    }
    if (p >= end) return false;
    ++p;
    return true;
  }
  bool value(Json &v, int depth) {
    if (depth > 64) return false;
    ws();
    if (p >= end) return false;
    if (*p == '{') {
      ++p;
      v.kind = Json::OBJ;
      ws();
      if (p < end && *p == '}') return ++p, true;
      for (;;) {
        ws();
        std::string k;
        if (!string(k)) return false;
        ws();
        if (p >= end || *p != ':') return false;
        ++p;
        Json c;
        if (!value(c, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(c));
        ws();
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == '}') return ++p, true;
        return false;
      }
    }
    if (*p == '[') {
      ++p;
      v.kind = Json::ARR;
      ws();
      if (p < end && *p == ']') return ++p, true;
      for (;;) {
        Json c;
        if (!value(c, depth + 1)) return false;
        v.arr.push_back(std::move(c));
        ws();
        if (p < end && *p == ',') { ++p; continue; }
        if (p < end && *p == ']') return ++p, true;
        return false;
      }
    }
    if (*p == '"') {
      v.kind = Json::STR;
      return string(v.str);
    }
    if (lit("true")) { v.kind = Json::BOOL; v.num = 1; return true; }
    if (lit("false")) { v.kind = Json::BOOL; return true; }
    if (lit("null")) { v.kind = Json::NUL; return true; }
    const std::string s(p, (size_t)(end - p) < 64 ? (size_t)(end - p) : 64);
    char *stop = nullptr;
    const double d = strtod(s.c_str(), &stop);
    if (stop == s.c_str()) return false;
    p += stop - s.c_str();
    v.kind = Json::NUM;
    v.num = d;
    return true;
  }
};

bool parse_json(const std::string &text, Json &out) {
  JsonParser jp{text.data(), text.data() + text.size()};
  if (!jp.value(out, 0)) return false;
  jp.ws();
  return jp.p == jp.end;
}

bool read_file(const std::string &path, std::string &out) {
  const int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return false;
  out.clear();
  char buf[1 << 16];
  for (;;) {
    const ssize_t n = read(fd, buf, sizeof buf);
    if (n < 0) { close(fd); return false; }
    if (n == 0) break;
    out.append(buf, (size_t)n);
  }
  close(fd);
  return true;
}

bool pread_all(int fd, void *dst, size_t n, size_t off) {
  uint8_t *d = static_cast<uint8_t *>(dst);
  while (n) {
    const ssize_t r = pread(fd, d, n, (off_t)off);
    if (r <= 0) return false;
    d += r;
    n -= (size_t)r;
    off += (size_t)r;
  }
  return true;
}

bool valid_utf8(const char *s) {
  const unsigned char *u = reinterpret_cast<const unsigned char *>(s);
  while (*u) {
    int n = *u < 0x80 ? 0 : (*u >> 5) == 6 ? 1 : (*u >> 4) == 14 ? 2 : (*u >> 3) == 30 ? 3 : -1;
    if (n < 0) return false;
    ++u;
    while (n--) {
      if ((*u & 0xC0) != 0x80) return false;
      ++u;
    }
  }
  return true;
}

// bf16::from_f32 (half 2.7.1, as c_ffi.rs:323 calls it): RNE, NaN made quiet.
uint16_t f32_to_bf16_host(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x0040u);
  return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// ---------------------------------------------------------------------------
// the source
// ---------------------------------------------------------------------------

struct TensorRef {
  std::string dtype;
  std::vector<int64_t> shape;
  size_t offset = 0, bytes = 0;  // absolute file offset, length
};

struct Shard {
  int fd = -1;
  size_t file_bytes = 0;
  std::unordered_map<std::string, TensorRef> tensors;
  ~Shard() {
    if (fd >= 0) close(fd);
  }
};

struct DeviceExpert {
  void *blob = nullptr;  // the tiled sections
  size_t bytes = 0;
  cascadia_int4_expert e{};
  uint32_t hidden = 0, inter = 0, group = 0, sdt = 0;
};

using ExpertKey = std::pair<uint32_t, uint32_t>;

size_t env_size(const char *name) {
  const char *v = getenv(name);
  if (!v || !*v) return 0;
  char *end = nullptr;
  const unsigned long long n = strtoull(v, &end, 10);
  return end && *end == '\0' ? (size_t)n : 0;
}

}  // namespace

struct CascadiaInt4Source {
  std::string dir;
  int device = 0;
  bool int4_bin = false;  // flat expert files (manifest experts_format "int4_bin")
  uint32_t bin_hidden = 0, bin_inter = 0;
  std::unordered_map<std::string, std::string> weight_map;  // tensor -> shard file
  std::unordered_map<std::string, std::unique_ptr<Shard>> shards;
  // the resident experts, most recently used first
  std::list<std::pair<ExpertKey, DeviceExpert>> lru;
  std::map<ExpertKey, std::list<std::pair<ExpertKey, DeviceExpert>>::iterator> experts;
  size_t max_experts = 0, max_bytes = 0, resident_bytes = 0;  // limits 0: unbounded
  uint64_t evictions = 0;
  hipStream_t stream = nullptr;
  uint16_t *x_dev = nullptr, *out_dev = nullptr;
  void *ws = nullptr;
  size_t io_elems = 0, ws_bytes = 0;
  std::mutex mu;
  // experts a prefetch is loading (guarded by mu); loaders wait on loaded_cv
  std::set<ExpertKey> inflight;
  std::condition_variable loaded_cv;
  // the prefetcher (runner.rs:282-360): a bounded queue, its thread, counters
  std::mutex qmu;
  std::condition_variable qcv;
  std::deque<ExpertKey> queue;
  std::thread worker;
  bool stop = false, busy = false;
  uint64_t submits = 0, drops = 0, processed = 0, loaded = 0;
};

namespace {

Shard *shard_of(CascadiaInt4Source *s, const std::string &file) {
  auto it = s->shards.find(file);
  if (it != s->shards.end()) return it->second.get();
  auto sh = std::make_unique<Shard>();
  sh->fd = open((s->dir + "/" + file).c_str(), O_RDONLY);
  if (sh->fd < 0) return nullptr;
  struct stat stt;
  if (fstat(sh->fd, &stt) != 0) return nullptr;
  sh->file_bytes = (size_t)stt.st_size;
  uint8_t hl[8];
  if (!pread_all(sh->fd, hl, 8, 0)) return nullptr;
  uint64_t n = 0;
  for (int i = 7; i >= 0; --i) n = (n << 8) | hl[i];
  // a header longer than the file is malformed (safetensors_source.rs:85-95)
  if (n > (1ull << 30) || n > sh->file_bytes - 8) return nullptr;
  std::string hdr(n, '\0');
  if (!pread_all(sh->fd, &hdr[0], n, 8)) return nullptr;
  Json j;
  if (!parse_json(hdr, j) || j.kind != Json::OBJ) return nullptr;
  const size_t data0 = 8 + n;
  for (const auto &kv : j.obj) {
    if (kv.first == "__metadata__") continue;
    const Json *off = kv.second.get("data_offsets");
    if (!off || off->kind != Json::ARR || off->arr.size() != 2) return nullptr;
    // as_u64().unwrap_or(0) (safetensors_source.rs:100-106): a negative,
    // fractional or non-numeric offset, or one past 2^53, reads as 0
    auto u64_or_0 = [](const Json &v) -> uint64_t {
      if (v.kind != Json::NUM || !(v.num >= 0.0) || v.num > 9007199254740992.0 ||
          v.num != (double)(uint64_t)v.num)
        return 0;
      return (uint64_t)v.num;
    };
    const uint64_t a = u64_or_0(off->arr[0]), b = u64_or_0(off->arr[1]);
    if (b < a) continue;  // safetensors_source.rs:107-109
    if (b > sh->file_bytes - data0) continue;  // past the end of the file: unreadable
    TensorRef t;
    t.offset = data0 + (size_t)a;
    t.bytes = (size_t)(b - a);
    if (const Json *d = kv.second.get("dtype")) t.dtype = d->str;
    if (const Json *sh2 = kv.second.get("shape"))
      for (const auto &e : sh2->arr) t.shape.push_back((int64_t)e.num);
    sh->tensors.emplace(kv.first, std::move(t));
  }
  Shard *raw = sh.get();
  s->shards.emplace(file, std::move(sh));
  return raw;
}

bool tensor(CascadiaInt4Source *s, const std::string &name, Shard **sh, const TensorRef **t) {
  auto it = s->weight_map.find(name);
  if (it == s->weight_map.end()) return false;
  *sh = shard_of(s, it->second);
  if (!*sh) return false;
  auto jt = (*sh)->tensors.find(name);
  if (jt == (*sh)->tensors.end()) return false;
  *t = &jt->second;
  return true;
}

// Drop the least recently used resident expert (after the handle's stream
// has drained: nothing in flight may still read it).  False when none is left.
bool evict_one(CascadiaInt4Source *s) {
  if (s->lru.empty()) return false;
  if (hipStreamSynchronize(s->stream) != hipSuccess) return false;
  auto &victim = s->lru.back();
  (void)hipFree(victim.second.blob);
  s->resident_bytes -= victim.second.bytes;
  s->experts.erase(victim.first);
  s->lru.pop_back();
  ++s->evictions;
  return true;
}

// Evict until one more expert of `bytes` fits the limits.
void make_room(CascadiaInt4Source *s, size_t bytes) {
  while (!s->lru.empty() &&
         ((s->max_experts && s->lru.size() + 1 > s->max_experts) ||
          (s->max_bytes && s->resident_bytes + bytes > s->max_bytes)))
    if (!evict_one(s)) break;
}

// hipMalloc that evicts resident experts and retries when HBM is full.
bool malloc_evicting(CascadiaInt4Source *s, void **p, size_t bytes) {
  for (;;) {
    if (hipMalloc(p, bytes) == hipSuccess) return true;
    (void)hipGetLastError();  // clear the failed allocation's error
    *p = nullptr;
    if (!evict_one(s)) return false;
  }
}

// Where one expert's six sections are (flat-blob order, format.rs:35-47) and
// its dims.  Resolving it may open shards, so it is made under the handle's
// lock; the reads it describes need no lock (shard descriptors stay open
// until the handle is destroyed).
struct ExpertPlan {
  uint32_t hidden = 0, inter = 0, group = 0, sdt = 0;
  int fd[6] = {-1, -1, -1, -1, -1, -1};
  size_t off[6] = {0, 0, 0, 0, 0, 0}, len[6] = {0, 0, 0, 0, 0, 0};
  int own_fd = -1;  // int4_bin: the expert file, opened for this plan
  ~ExpertPlan() {
    if (own_fd >= 0) close(own_fd);
  }
};

// Expert (L, E) of a safetensors directory: 0, or -2.
int plan_safetensors_expert(CascadiaInt4Source *s, uint32_t layer, uint32_t expert,
                            ExpertPlan *p) {
  const std::string base = "language_model.model.layers." + std::to_string(layer) +
                           ".mlp.experts." + std::to_string(expert) + ".";
  static const char *kNames[6] = {"gate_proj.weight_packed", "gate_proj.weight_scale",
                                  "up_proj.weight_packed",   "up_proj.weight_scale",
                                  "down_proj.weight_packed", "down_proj.weight_scale"};
  Shard *sh[6];
  const TensorRef *t[6];
  for (int i = 0; i < 6; ++i)
    if (!tensor(s, base + kNames[i], &sh[i], &t[i])) return -2;
  // dims from the gate tensors: packed [inter, hidden / 8] int32 (or bytes of
  // inter * hidden / 2), scales [inter, hidden / G]
  if (t[0]->shape.size() != 2 || t[1]->shape.size() != 2) return -2;
  const int64_t inter = t[0]->shape[0];
  const int64_t hidden = t[0]->dtype == "U8" || t[0]->dtype == "I8" ? t[0]->shape[1] * 2
                                                                     : t[0]->shape[1] * 8;
  if (inter <= 0 || hidden <= 0 || t[1]->shape[0] != inter || t[1]->shape[1] <= 0 ||
      hidden % t[1]->shape[1])
    return -2;
  const int64_t group = hidden / t[1]->shape[1];
  const size_t pin = (size_t)inter * hidden / 2, sin = (size_t)inter * (hidden / group) * 2;
  const size_t pdn = (size_t)hidden * inter / 2, sdn = (size_t)hidden * (inter / group) * 2;
  const size_t want[6] = {pin, sin, pin, sin, pdn, sdn};
  for (int i = 0; i < 6; ++i)
    if (t[i]->bytes != want[i]) return -2;
  if (group % 32 || inter % group || inter > (1 << 30) || hidden > (1 << 30)) return -2;
  for (int i = 0; i < 6; ++i) {
    p->fd[i] = sh[i]->fd;
    p->off[i] = t[i]->offset;
    p->len[i] = want[i];
  }
  p->hidden = (uint32_t)hidden;
  p->inter = (uint32_t)inter;
  p->group = (uint32_t)group;
  p->sdt = t[1]->dtype == "F16" ? CASCADIA_INT4_SCALE_F16 : CASCADIA_INT4_SCALE_BF16;
  return 0;
}

// experts/layer_LL/expert_EEE.bin (manifest.rs:137-142): the flat blob of
// format.rs:35-47 at the manifest's dims, G 32, bf16 scales: 0, or -2.
int plan_bin_expert(CascadiaInt4Source *s, uint32_t layer, uint32_t expert, ExpertPlan *p) {
  char name[64];
  snprintf(name, sizeof name, "/experts/layer_%02u/expert_%03u.bin", layer, expert);
  const int fd = open((s->dir + name).c_str(), O_RDONLY);
  if (fd < 0) return -2;
  p->own_fd = fd;
  const size_t flat = cascadia_int4_expert_bytes(s->bin_hidden, s->bin_inter, 32);
  struct stat stt;
  if (!flat || fstat(fd, &stt) != 0 || (size_t)stt.st_size != flat) return -2;
  p->fd[0] = fd;
  p->off[0] = 0;
  p->len[0] = flat;  // one read of the whole blob
  p->hidden = s->bin_hidden;
  p->inter = s->bin_inter;
  p->group = 32;
  p->sdt = CASCADIA_INT4_SCALE_BF16;
  return 0;
}

int plan_expert(CascadiaInt4Source *s, uint32_t layer, uint32_t expert, ExpertPlan *p) {
  return s->int4_bin ? plan_bin_expert(s, layer, expert, p)
                     : plan_safetensors_expert(s, layer, expert, p);
}

// The planned sections into a pinned host buffer *host (allocated here, in
// the flat-blob order): 0, -2 (a short read), -3 (no pinned memory).
int read_plan(const ExpertPlan &p, void **host) {
  size_t flat = 0;
  for (int i = 0; i < 6; ++i) flat += p.len[i];
  if (hipHostMalloc(host, flat, hipHostMallocDefault) != hipSuccess) {
    *host = nullptr;
    return -3;
  }
  size_t off = 0;
  for (int i = 0; i < 6; ++i) {
    if (!p.len[i]) continue;
    if (!pread_all(p.fd[i], static_cast<uint8_t *>(*host) + off, p.len[i], p.off[i])) {
      (void)hipHostFree(*host);
      *host = nullptr;
      return -2;
    }
    off += p.len[i];
  }
  return 0;
}

// Upload the flat blob at `host` to dflat, tile it into dtiled on `st` and
// wait: 0, -2, -3.  dflat / dtiled are the caller's.
int upload_expert(const ExpertPlan &p, const void *host, void *dflat, void *dtiled,
                  cascadia_int4_expert *tiled_out, hipStream_t st) {
  const size_t flat = cascadia_int4_expert_bytes(p.hidden, p.inter, p.group);
  cascadia_int4_expert src{};
  if (hipMemcpyAsync(dflat, host, flat, hipMemcpyHostToDevice, st) != hipSuccess) return -3;
  if (cascadia_int4_expert_from_flat(static_cast<uint8_t *>(dflat), p.hidden, p.inter, p.group,
                                     &src) != 0)
    return -2;
  if (cascadia_int4_tile_expert(p.hidden, p.inter, p.group, &src, static_cast<uint8_t *>(dtiled),
                                tiled_out, st) != 0)
    return -3;
  return hipStreamSynchronize(st) == hipSuccess ? 0 : -3;
}

// Make an uploaded expert resident, most recently used first.
DeviceExpert *insert_expert(CascadiaInt4Source *s, const ExpertKey &key, const ExpertPlan &p,
                            void *dtiled, const cascadia_int4_expert &e) {
  DeviceExpert de;
  de.blob = dtiled;
  de.bytes = cascadia_int4_expert_tiled_bytes(p.hidden, p.inter, p.group);
  de.e = e;
  de.hidden = p.hidden;
  de.inter = p.inter;
  de.group = p.group;
  de.sdt = p.sdt;
  s->lru.emplace_front(key, de);
  s->experts[key] = s->lru.begin();
  s->resident_bytes += de.bytes;
  return &s->lru.front().second;
}

// 0, -2 (the expert's data missing or inconsistent), -3 (HIP failure or no
// room in HBM even with every other expert evicted).  The caller holds lk on
// the handle's lock; an expert a prefetch is loading is waited for, not read
// a second time.
int load_expert(CascadiaInt4Source *s, uint32_t layer, uint32_t expert, DeviceExpert **out,
                std::unique_lock<std::mutex> &lk) {
  const ExpertKey key = std::make_pair(layer, expert);
  s->loaded_cv.wait(lk, [&] { return s->inflight.count(key) == 0; });
  auto it = s->experts.find(key);
  if (it != s->experts.end()) {
    s->lru.splice(s->lru.begin(), s->lru, it->second);  // most recently used
    *out = &it->second->second;
    return 0;
  }
  ExpertPlan p;
  int rc = plan_expert(s, layer, expert, &p);
  void *host = nullptr;
  if (!rc) rc = read_plan(p, &host);
  if (rc) return rc;
  const size_t flat = cascadia_int4_expert_bytes(p.hidden, p.inter, p.group);
  const size_t tiled = cascadia_int4_expert_tiled_bytes(p.hidden, p.inter, p.group);
  if (!flat || !tiled) {
    (void)hipHostFree(host);
    return -2;
  }
  make_room(s, tiled);
  void *dflat = nullptr, *dtiled = nullptr;
  cascadia_int4_expert e{};
  if (!malloc_evicting(s, &dtiled, tiled) || !malloc_evicting(s, &dflat, flat)) rc = -3;
  if (!rc) rc = upload_expert(p, host, dflat, dtiled, &e, s->stream);
  (void)hipHostFree(host);
  if (dflat) (void)hipFree(dflat);
  if (rc) {
    if (dtiled) (void)hipFree(dtiled);
    return rc;
  }
  *out = insert_expert(s, key, p, dtiled, e);
  return 0;
}

// One prefetch request on the prefetcher's thread: the disk read and the
// upload run without the handle's lock (foreground calls go on meanwhile;
// one for this expert waits for it), the allocation and the insertion with
// it.  Errors are dropped: the expert then loads on first use, as a miss.
// True when the expert was loaded.
bool prefetch_one(CascadiaInt4Source *s, const ExpertKey &key, hipStream_t ps) {
  ExpertPlan p;
  {
    std::lock_guard<std::mutex> lk(s->mu);
    if (s->experts.count(key) || s->inflight.count(key)) return false;  // resident or loading
    if (plan_expert(s, key.first, key.second, &p) != 0) return false;
    s->inflight.insert(key);
  }
  void *host = nullptr, *dflat = nullptr, *dtiled = nullptr;
  cascadia_int4_expert e{};
  int rc = read_plan(p, &host);
  const size_t flat = cascadia_int4_expert_bytes(p.hidden, p.inter, p.group);
  const size_t tiled = cascadia_int4_expert_tiled_bytes(p.hidden, p.inter, p.group);
  if (!rc && (!flat || !tiled)) rc = -2;
  if (!rc) {
    std::lock_guard<std::mutex> lk(s->mu);
    make_room(s, tiled);
    if (!malloc_evicting(s, &dtiled, tiled) || !malloc_evicting(s, &dflat, flat)) rc = -3;
  }
  if (!rc) rc = upload_expert(p, host, dflat, dtiled, &e, ps);
  if (host) (void)hipHostFree(host);
  if (dflat) (void)hipFree(dflat);
  std::lock_guard<std::mutex> lk(s->mu);
  if (rc) {
    if (dtiled) (void)hipFree(dtiled);
  } else {
    make_room(s, tiled);  // limits may have been reached while it loaded
    insert_expert(s, key, p, dtiled, e);
  }
  s->inflight.erase(key);
  s->loaded_cv.notify_all();
  return rc == 0;
}

// The prefetcher's thread: requests in queue order until the handle stops.
void prefetch_loop(CascadiaInt4Source *s) {
  const bool dev_ok = hipSetDevice(s->device) == hipSuccess;
  hipStream_t ps = nullptr;
  const bool ok = dev_ok && hipStreamCreateWithFlags(&ps, hipStreamNonBlocking) == hipSuccess;
  for (;;) {
    ExpertKey key;
    {
      std::unique_lock<std::mutex> q(s->qmu);
      s->qcv.wait(q, [&] { return s->stop || !s->queue.empty(); });
      if (s->stop) break;
      key = s->queue.front();
      s->queue.pop_front();
      s->busy = true;
    }
    const bool loaded = ok && prefetch_one(s, key, ps);
    {
      std::lock_guard<std::mutex> q(s->qmu);
      ++s->processed;
      if (loaded) ++s->loaded;
      s->busy = false;
    }
    s->qcv.notify_all();
  }
  if (ps) (void)hipStreamDestroy(ps);
}

// Make the handle's device current for the call; restore the caller's after.
struct DeviceScope {
  int prev = -1;
  bool ok = false;
  explicit DeviceScope(int dev) {
    if (hipGetDevice(&prev) != hipSuccess) return;
    ok = prev == dev || hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceScope() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

}  // namespace

extern "C" {

int cascadia_int4_open_source(const char *model_dir, CascadiaInt4Source **out_handle) {
  if (!model_dir || !out_handle) return -1;
  if (!valid_utf8(model_dir)) return -2;
  auto s = std::make_unique<CascadiaInt4Source>();
  s->dir = model_dir;
  std::string text;
  Json man;
  const Json *fmt = nullptr;
  if (read_file(s->dir + "/manifest.json", text) && parse_json(text, man) &&
      (fmt = man.get("experts_format")) && fmt->kind == Json::STR && fmt->str == "int4_bin") {
    // the flat-expert layout (manifest.rs:21-80: hidden_size, expert_intermediate)
    const Json *hs = man.get("hidden_size"), *ei = man.get("expert_intermediate");
    if (!hs || hs->kind != Json::NUM || !(hs->num >= 32) || hs->num > (double)(1 << 20))
      return -3;
    s->int4_bin = true;
    s->bin_hidden = (uint32_t)hs->num;
    if (!ei) {
      // no expert_intermediate: the K2.6 runner's reader, whose
      // ExpertWeights::open is fixed to HIDDEN x INTERMEDIATE = 7168 x 2048
      // (runner.rs:697-705, format.rs:63, lib.rs:71-78)
      if (s->bin_hidden != 7168u) return -3;
      s->bin_inter = 2048u;
    } else {
      // ov_moe.rs:452-457: int4_bin requires expert_intermediate > 0
      if (ei->kind != Json::NUM || !(ei->num >= 1) || ei->num > (double)(1u << 20)) return -3;
      s->bin_inter = (uint32_t)ei->num;
    }
    if (s->bin_hidden % 32 || s->bin_inter % 32) return -3;
  } else {
    Json idx;
    if (!read_file(s->dir + "/model.safetensors.index.json", text) || !parse_json(text, idx))
      return -3;
    const Json *wm = idx.get("weight_map");
    if (!wm || wm->kind != Json::OBJ) return -3;
    for (const auto &kv : wm->obj)
      if (kv.second.kind == Json::STR) s->weight_map.emplace(kv.first, kv.second.str);
  }
  s->max_experts = env_size("CASCADIA_INT4_MAX_CACHED_EXPERTS");
  s->max_bytes = env_size("CASCADIA_INT4_EXPERT_CACHE_BYTES");
  if (hipGetDevice(&s->device) != hipSuccess) return -3;
  if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) return -3;
  *out_handle = s.release();
  return 0;
}

void cascadia_int4_destroy_source(CascadiaInt4Source *handle) {
  if (!handle) return;
  {  // stop the prefetcher: queued requests are dropped, a load in progress finishes
    std::lock_guard<std::mutex> q(handle->qmu);
    handle->stop = true;
    handle->queue.clear();
  }
  handle->qcv.notify_all();
  if (handle->worker.joinable()) handle->worker.join();
  {
    DeviceScope ds(handle->device);
    if (handle->stream) (void)hipStreamSynchronize(handle->stream);
    for (auto &kv : handle->lru) (void)hipFree(kv.second.blob);
    if (handle->x_dev) (void)hipFree(handle->x_dev);
    if (handle->out_dev) (void)hipFree(handle->out_dev);
    if (handle->ws) (void)hipFree(handle->ws);
    if (handle->stream) (void)hipStreamDestroy(handle->stream);
  }
  delete handle;
}

int cascadia_int4_prewarm(CascadiaInt4Source *handle, uint32_t layer, uint32_t expert) {
  if (!handle) return -1;
  std::unique_lock<std::mutex> lk(handle->mu);
  DeviceScope ds(handle->device);
  if (!ds.ok) return -3;
  DeviceExpert *de = nullptr;
  return load_expert(handle, layer, expert, &de, lk);
}

int cascadia_int4_prefetch(CascadiaInt4Source *handle, uint32_t layer, uint32_t expert) {
  if (!handle) return -1;
  constexpr size_t kQueue = 4096;  // the runner's sync_channel bound (runner.rs:296-300)
  {
    std::lock_guard<std::mutex> q(handle->qmu);
    if (handle->stop) return 0;
    if (!handle->worker.joinable()) {
      try {
        handle->worker = std::thread(prefetch_loop, handle);
      } catch (...) {
        ++handle->drops;  // no thread: the request is dropped, as on overflow
        return 0;
      }
    }
    if (handle->queue.size() >= kQueue) {
      ++handle->drops;
      return 0;
    }
    handle->queue.emplace_back(layer, expert);
    ++handle->submits;
  }
  handle->qcv.notify_all();
  return 0;
}

int cascadia_int4_prefetch_wait(CascadiaInt4Source *handle) {
  if (!handle) return -1;
  std::unique_lock<std::mutex> q(handle->qmu);
  handle->qcv.wait(q, [&] { return handle->stop || (handle->queue.empty() && !handle->busy); });
  return 0;
}

int cascadia_int4_prefetch_stats(CascadiaInt4Source *handle, uint64_t *submits, uint64_t *drops,
                                 uint64_t *processed, uint64_t *loaded) {
  if (!handle) return -1;
  std::lock_guard<std::mutex> q(handle->qmu);
  if (submits) *submits = handle->submits;
  if (drops) *drops = handle->drops;
  if (processed) *processed = handle->processed;
  if (loaded) *loaded = handle->loaded;
  return 0;
}

int cascadia_int4_expert_forward(CascadiaInt4Source *handle, uint32_t layer, uint32_t expert,
                                 const float *x_f32, float *out_f32) {
  if (!handle || !x_f32 || !out_f32) return -1;
  std::unique_lock<std::mutex> lk(handle->mu);
  DeviceScope ds(handle->device);
  if (!ds.ok) return -3;
  DeviceExpert *de = nullptr;
  if (int rc = load_expert(handle, layer, expert, &de, lk)) return rc;
  const uint32_t h = de->hidden;
  const size_t need_ws = cascadia_int4_ffn_workspace_bytes(h, de->inter, de->group, 1);
  if (handle->io_elems < h) {
    if (handle->x_dev) (void)hipFree(handle->x_dev);
    if (handle->out_dev) (void)hipFree(handle->out_dev);
    handle->x_dev = handle->out_dev = nullptr;
    handle->io_elems = 0;
    if (!malloc_evicting(handle, reinterpret_cast<void **>(&handle->x_dev), (size_t)h * 2) ||
        !malloc_evicting(handle, reinterpret_cast<void **>(&handle->out_dev), (size_t)h * 2))
      return -3;
    handle->io_elems = h;
  }
  if (handle->ws_bytes < need_ws) {
    if (handle->ws) (void)hipFree(handle->ws);
    handle->ws = nullptr;
    handle->ws_bytes = 0;
    if (!malloc_evicting(handle, &handle->ws, need_ws)) return -3;
    handle->ws_bytes = need_ws;
  }
  // the expert may have been evicted to make room for the buffers: reload
  if (int rc = load_expert(handle, layer, expert, &de, lk)) return rc;
  std::vector<uint16_t> xb(h), ob(h);
  for (uint32_t i = 0; i < h; ++i) xb[i] = f32_to_bf16_host(x_f32[i]);  // c_ffi.rs:323
  if (hipMemcpyAsync(handle->x_dev, xb.data(), (size_t)h * 2, hipMemcpyHostToDevice,
                     handle->stream) != hipSuccess)
    return -3;
  if (cascadia_int4_expert_forward_device(h, de->inter, de->group, de->sdt, &de->e, handle->x_dev,
                                          1, handle->out_dev, handle->ws, handle->stream) != 0)
    return -3;
  if (hipMemcpyAsync(ob.data(), handle->out_dev, (size_t)h * 2, hipMemcpyDeviceToHost,
                     handle->stream) != hipSuccess ||
      hipStreamSynchronize(handle->stream) != hipSuccess)
    return -3;
  for (uint32_t i = 0; i < h; ++i) {  // bf16 -> f32, c_ffi.rs:336-338
    const uint32_t b = (uint32_t)ob[i] << 16;
    memcpy(&out_f32[i], &b, 4);
  }
  return 0;
}

int cascadia_int4_source_set_cache_limits(CascadiaInt4Source *handle, uint64_t max_experts,
                                          uint64_t max_bytes) {
  if (!handle) return -1;
  std::lock_guard<std::mutex> lk(handle->mu);
  DeviceScope ds(handle->device);
  if (!ds.ok) return -3;
  handle->max_experts = (size_t)max_experts;
  handle->max_bytes = (size_t)max_bytes;
  while (!handle->lru.empty() &&
         ((handle->max_experts && handle->lru.size() > handle->max_experts) ||
          (handle->max_bytes && handle->resident_bytes > handle->max_bytes)))
    if (!evict_one(handle)) return -3;
  return 0;
}

int cascadia_int4_source_cache_stats(CascadiaInt4Source *handle, uint64_t *cached,
                                     uint64_t *evictions, uint64_t *resident_bytes) {
  if (!handle) return -1;
  std::lock_guard<std::mutex> lk(handle->mu);
  if (cached) *cached = handle->lru.size();
  if (evictions) *evictions = handle->evictions;
  if (resident_bytes) *resident_bytes = handle->resident_bytes;
  return 0;
}

}  // extern "C"
