// Checkpoint files of the training step, host code only: the safetensors
// codec and the staged directory write of Model::save (crates/sejong-model/
// src/lib.rs:395-538).
//
// safetensors is the format of the `safetensors` crate the reference pins
// (Cargo.lock: 0.8.0; save_tensors / load_tensors, model lib.rs:456-538):
//   8-byte little-endian header length N,
//   N bytes of compact JSON {"<name>":{"dtype":"F32","shape":[..],
//     "data_offsets":[begin,end]},...} -- tensors ordered by dtype (wider
//     first) and then by name, byte-wise -- padded with spaces to a
//     multiple of 8,
//   the tensors' little-endian bytes back to back in that order.
// The checkpoint tensors are F32 (parameter masters, AdamW moments, the SGD
// state words), so the order is the byte-wise name order.
#include <errno.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#include <algorithm>
#include <string>
#include <vector>

#include "common.h"

namespace {

struct Spec {
  std::string name;
  std::vector<long> shape;
  const float* data;
  size_t count;
};

// serde_json string escaping (quote, backslash, control characters)
std::string json_string(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"') o += "\\\"";
    else if (c == '\\') o += "\\\\";
    else if (c == '\n') o += "\\n";
    else if (c == '\r') o += "\\r";
    else if (c == '\t') o += "\\t";
    else if (c == '\b') o += "\\b";
    else if (c == '\f') o += "\\f";
    else if (c < 0x20) {
      char b[8];
      snprintf(b, sizeof b, "\\u%04x", c);
      o += b;
    } else {
      o += (char)c;
    }
  }
  return o + "\"";
}

int write_all(FILE* f, const void* p, size_t n, const std::string& path) {
  if (n && fwrite(p, 1, n, f) != n) return sjh::fail(SJ_ERR_IO, "write %s: %s", path.c_str(), strerror(errno));
  return SJ_OK;
}

int write_safetensors(const std::string& path, std::vector<Spec> specs) {
  std::sort(specs.begin(), specs.end(), [](const Spec& a, const Spec& b) { return a.name < b.name; });
  for (size_t i = 1; i < specs.size(); i++)
    if (specs[i].name == specs[i - 1].name) return sjh::fail(SJ_ERR_INVALID, "safetensors: duplicate tensor %s",
                                                             specs[i].name.c_str());
  std::string h = "{";
  size_t off = 0;
  for (size_t i = 0; i < specs.size(); i++) {
    const Spec& s = specs[i];
    if (i) h += ",";
    h += json_string(s.name) + ":{\"dtype\":\"F32\",\"shape\":[";
    for (size_t k = 0; k < s.shape.size(); k++) h += (k ? "," : "") + std::to_string(s.shape[k]);
    const size_t end = off + 4 * s.count;
    h += "],\"data_offsets\":[" + std::to_string(off) + "," + std::to_string(end) + "]}";
    off = end;
  }
  h += "}";
  while (h.size() % 8) h += ' ';
  FILE* f = fopen(path.c_str(), "wb");
  if (!f) return sjh::fail(SJ_ERR_IO, "create %s: %s", path.c_str(), strerror(errno));
  uint8_t len[8];
  for (int i = 0; i < 8; i++) len[i] = (uint8_t)((uint64_t)h.size() >> (8 * i));
  int st = write_all(f, len, 8, path);
  if (!st) st = write_all(f, h.data(), h.size(), path);
  for (size_t i = 0; i < specs.size() && !st; i++) st = write_all(f, specs[i].data, 4 * specs[i].count, path);
  if (fclose(f) != 0 && !st) st = sjh::fail(SJ_ERR_IO, "close %s: %s", path.c_str(), strerror(errno));
  return st;
}

int specs_from(long n, const char* const* names, const long* ranks, const long* dims, const float* const* data,
               std::vector<Spec>& out) {
  long di = 0;
  for (long i = 0; i < n; i++) {
    SJ_REQUIRE(names && names[i] && ranks && ranks[i] >= 0 && ranks[i] <= 8 && data && data[i],
               "checkpoint: tensor %ld: name, rank and data required", i);
    Spec s;
    s.name = names[i];
    s.data = data[i];
    s.count = 1;
    for (long k = 0; k < ranks[i]; k++) {
      SJ_REQUIRE(dims[di] >= 0, "checkpoint: tensor %s: negative dimension", names[i]);
      s.shape.push_back(dims[di]);
      s.count *= (size_t)dims[di++];
    }
    out.push_back(std::move(s));
  }
  return SJ_OK;
}

bool exists(const std::string& p) {
  struct stat sb;
  return stat(p.c_str(), &sb) == 0;
}

int make_dirs(const std::string& p) {
  if (p.empty() || exists(p)) return SJ_OK;
  size_t cut = p.find_last_of('/');
  if (cut != std::string::npos && cut > 0) {
    int st = make_dirs(p.substr(0, cut));
    if (st) return st;
  }
  if (mkdir(p.c_str(), 0777) != 0 && errno != EEXIST)
    return sjh::fail(SJ_ERR_IO, "create directory %s: %s", p.c_str(), strerror(errno));
  return SJ_OK;
}

void remove_tree(const std::string& dir) {
  for (const char* f : {"weights.safetensors", "optimizer.safetensors", "manifest.json"})
    unlink((dir + "/" + f).c_str());
  rmdir(dir.c_str());
}

// ---------------------------------------------------------------- reader
struct Json {  // the subset a safetensors header uses
  enum Kind { OBJ, ARR, STR, NUM } kind = NUM;
  std::string s;
  double num = 0;
  std::vector<std::pair<std::string, Json>> obj;
  std::vector<Json> arr;
  const Json* get(const std::string& k) const {
    for (const auto& kv : obj)
      if (kv.first == k) return &kv.second;
    return nullptr;
  }
};

struct Parser {
  const char* p;
  const char* e;
  bool ok = true;
  void ws() {
    while (p < e && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) p++;
  }
  bool str(std::string& o) {
    if (p >= e || *p != '"') return false;
    p++;
    while (p < e && *p != '"') {
      if (*p == '\\') {
        if (++p >= e) return false;
        switch (*p) {
          case 'n': o += '\n'; break;
          case 't': o += '\t'; break;
          case 'r': o += '\r'; break;
          case 'b': o += '\b'; break;
          case 'f': o += '\f'; break;
          case 'u': {
            if (e - p < 5) return false;
            unsigned v = 0;
            for (int i = 1; i <= 4; i++) {
              char c = p[i];
              v = v * 16 + (unsigned)(c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10
                                                                  : c >= 'A' && c <= 'F' ? c - 'A' + 10 : 0);
            }
            if (v < 0x80) o += (char)v;
            else if (v < 0x800) { o += (char)(0xc0 | (v >> 6)); o += (char)(0x80 | (v & 0x3f)); }
            else { o += (char)(0xe0 | (v >> 12)); o += (char)(0x80 | ((v >> 6) & 0x3f)); o += (char)(0x80 | (v & 0x3f)); }
            p += 4;
            break;
          }
          default: o += *p;
        }
        p++;
      } else {
        o += *p++;
      }
    }
    if (p >= e) return false;
    p++;
    return true;
  }
  bool value(Json& v, int depth = 0) {
    if (depth > 8) return false;
    ws();
    if (p >= e) return false;
    if (*p == '{') {
      v.kind = Json::OBJ;
      p++;
      ws();
      if (p < e && *p == '}') { p++; return true; }
      for (;;) {
        std::string k;
        ws();
        if (!str(k)) return false;
        ws();
        if (p >= e || *p != ':') return false;
        p++;
        Json c;
        if (!value(c, depth + 1)) return false;
        v.obj.emplace_back(std::move(k), std::move(c));
        ws();
        if (p < e && *p == ',') { p++; continue; }
        if (p < e && *p == '}') { p++; return true; }
        return false;
      }
    }
    if (*p == '[') {
      v.kind = Json::ARR;
      p++;
      ws();
      if (p < e && *p == ']') { p++; return true; }
      for (;;) {
        Json c;
        if (!value(c, depth + 1)) return false;
        v.arr.push_back(std::move(c));
        ws();
        if (p < e && *p == ',') { p++; continue; }
        if (p < e && *p == ']') { p++; return true; }
        return false;
      }
    }
    if (*p == '"') {
      v.kind = Json::STR;
      return str(v.s);
    }
    v.kind = Json::NUM;
    const char* q = p;
    while (p < e && (isdigit((unsigned char)*p) || *p == '-' || *p == '+' || *p == '.' || *p == 'e' || *p == 'E')) p++;
    if (p == q) return false;
    v.num = strtod(std::string(q, p).c_str(), nullptr);
    return true;
  }
};

struct Header {
  std::string text;
  Json root;
  size_t data_start = 0, file_size = 0;
};

int read_header(const char* path, Header& h) {
  FILE* f = fopen(path, "rb");
  if (!f) return sjh::fail(SJ_ERR_IO, "open %s: %s", path, strerror(errno));
  uint8_t len[8];
  int st = SJ_OK;
  if (fread(len, 1, 8, f) != 8) st = sjh::fail(SJ_ERR_IO, "%s: not a safetensors file (short)", path);
  uint64_t n = 0;
  for (int i = 0; i < 8 && !st; i++) n |= (uint64_t)len[i] << (8 * i);
  fseek(f, 0, SEEK_END);
  const long size = ftell(f);
  if (!st && (n > (uint64_t)100000000 || 8 + n > (uint64_t)size))
    st = sjh::fail(SJ_ERR_IO, "%s: invalid safetensors header length", path);
  if (!st) {
    h.text.resize(n);
    fseek(f, 8, SEEK_SET);
    if (fread(&h.text[0], 1, n, f) != n) st = sjh::fail(SJ_ERR_IO, "%s: short header", path);
  }
  fclose(f);
  if (st) return st;
  Parser P{h.text.data(), h.text.data() + h.text.size()};
  if (!P.value(h.root) || h.root.kind != Json::OBJ)
    return sjh::fail(SJ_ERR_IO, "%s: invalid safetensors header", path);
  h.data_start = 8 + n;
  h.file_size = (size_t)size;
  // every tensor's byte range lies inside the data section
  for (const auto& kv : h.root.obj) {
    if (kv.first == "__metadata__") continue;
    const Json* off = kv.second.get("data_offsets");
    if (!off || off->kind != Json::ARR || off->arr.size() != 2 || off->arr[0].num < 0 ||
        off->arr[1].num < off->arr[0].num || h.data_start + (size_t)off->arr[1].num > h.file_size)
      return sjh::fail(SJ_ERR_IO, "%s: tensor %s: invalid data offsets", path, kv.first.c_str());
  }
  return SJ_OK;
}

}  // namespace

/* -------------------------------------------------------------- C ABI */

extern "C" int sj_safetensors_write(const char* path, long count, const char* const* names, const long* ranks,
                                    const long* dims, const float* const* data) {
  SJ_REQUIRE(path && count >= 0, "safetensors: path");
  std::vector<Spec> specs;
  if (int st = specs_from(count, names, ranks, dims, data, specs)) return st;
  return write_safetensors(path, std::move(specs));
}

extern "C" int sj_safetensors_header(const char* path, char* out, size_t capacity, size_t* length) {
  SJ_REQUIRE(path, "safetensors: path");
  Header h;
  if (int st = read_header(path, h)) return st;
  if (length) *length = h.text.size();
  if (out) {
    SJ_REQUIRE(capacity > h.text.size(), "safetensors: header needs %zu bytes", h.text.size() + 1);
    memcpy(out, h.text.data(), h.text.size());
    out[h.text.size()] = 0;
  }
  return SJ_OK;
}

extern "C" int sj_safetensors_read(const char* path, const char* name, float* out, long count) {
  SJ_REQUIRE(path && name && out && count >= 0, "safetensors: arguments");
  Header h;
  if (int st = read_header(path, h)) return st;
  const Json* t = h.root.get(name);
  if (!t) return sjh::fail(SJ_ERR_INVALID, "missing tensor %s", name);
  const Json* dt = t->get("dtype");
  const Json* shape = t->get("shape");
  const Json* off = t->get("data_offsets");
  long n = 1;
  if (shape && shape->kind == Json::ARR)
    for (const Json& d : shape->arr) n *= (long)d.num;
  if (!dt || dt->s != "F32" || !shape || n != count || (size_t)(off->arr[1].num - off->arr[0].num) != 4 * (size_t)n)
    return sjh::fail(SJ_ERR_INVALID, "tensor %s shape or dtype differs from configuration", name);
  FILE* f = fopen(path, "rb");
  if (!f) return sjh::fail(SJ_ERR_IO, "open %s: %s", path, strerror(errno));
  fseek(f, (long)(h.data_start + (size_t)off->arr[0].num), SEEK_SET);
  const size_t got = fread(out, 4, (size_t)n, f);
  fclose(f);
  if (got != (size_t)n) return sjh::fail(SJ_ERR_IO, "%s: short read of %s", path, name);
  for (long i = 0; i < n; i++)
    if (!isfinite(out[i])) return sjh::fail(SJ_ERR_INVALID, "tensor %s contains nonfinite values", name);
  return SJ_OK;
}

extern "C" int sj_checkpoint_save(const char* directory, const char* manifest_json, long n_weights,
                                  const char* const* weight_names, const long* weight_ranks, const long* weight_dims,
                                  const float* const* weight_data, long n_optimizer,
                                  const char* const* optimizer_names, const long* optimizer_ranks,
                                  const long* optimizer_dims, const float* const* optimizer_data) {
  SJ_REQUIRE(directory && directory[0] && manifest_json, "checkpoint: directory and manifest required");
  std::string dir(directory);
  while (dir.size() > 1 && dir.back() == '/') dir.pop_back();
  if (exists(dir)) return sjh::fail(SJ_ERR_INVALID, "artifact destination already exists: %s", dir.c_str());
  const size_t cut = dir.find_last_of('/');
  const std::string parent = cut == std::string::npos ? "." : (cut == 0 ? "/" : dir.substr(0, cut));
  const std::string name = cut == std::string::npos ? dir : dir.substr(cut + 1);
  SJ_REQUIRE(!name.empty() && name != "." && name != "..", "artifact destination requires a directory name");
  std::vector<Spec> ws, os;
  if (int st = specs_from(n_weights, weight_names, weight_ranks, weight_dims, weight_data, ws)) return st;
  if (n_optimizer > 0)
    if (int st = specs_from(n_optimizer, optimizer_names, optimizer_ranks, optimizer_dims, optimizer_data, os))
      return st;
  if (int st = make_dirs(parent)) return st;
  const std::string staging = parent + "/." + name + "." + std::to_string((long)getpid()) + ".tmp";
  if (mkdir(staging.c_str(), 0777) != 0)
    return sjh::fail(SJ_ERR_IO, "create %s: %s", staging.c_str(), strerror(errno));
  int st = write_safetensors(staging + "/weights.safetensors", std::move(ws));
  if (!st && n_optimizer > 0) st = write_safetensors(staging + "/optimizer.safetensors", std::move(os));
  if (!st) {
    FILE* f = fopen((staging + "/manifest.json").c_str(), "wb");
    if (!f) {
      st = sjh::fail(SJ_ERR_IO, "create manifest: %s", strerror(errno));
    } else {
      st = write_all(f, manifest_json, strlen(manifest_json), "manifest.json");
      if (fclose(f) != 0 && !st) st = sjh::fail(SJ_ERR_IO, "close manifest: %s", strerror(errno));
    }
  }
  if (!st && rename(staging.c_str(), dir.c_str()) != 0)
    st = sjh::fail(SJ_ERR_IO, "rename %s -> %s: %s", staging.c_str(), dir.c_str(), strerror(errno));
  if (st) remove_tree(staging);
  return st;
}
