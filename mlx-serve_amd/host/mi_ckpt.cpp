// Quantized-checkpoint loader behind include/mi_ckpt.h.
//
// Restates, for the tensors a quantized linear layer needs, what the reference
// does at model load:
//   config.json "quantization" block        src/model.zig:1480-1505 (defaults :152-156)
//   directory scan + per-file load          src/model.zig:2946-3027, 3089-3146
//   f16 side-tensor / 1-D narrowing         src/model.zig:3057-3084
//   vision/audio key filter                 src/model.zig:3148-3185
//   linear binding (.weight/.scales/.biases) src/transformer.zig:21068-21153
//   per-weight params                        src/transformer.zig:16657-16665 (detectQuantBits),
//                                            :16763-16782 (affineParamsFromGeometry),
//                                            :16850-16874 (fpQuantModeFor / fpParamsFromGeometry),
//                                            :16876-16924 (computeQuantParams)
// mlx_load_safetensors itself (MLX, un-vendored) is restated from the published
// safetensors layout: an 8-byte little-endian header length, a JSON header of
// {name: {dtype, shape, data_offsets:[begin,end]}} plus an optional
// "__metadata__" object, then the byte buffer the offsets index.
#include "../../include/mi_ckpt.h"

#include <dirent.h>
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace mi {
int report_error(int code, const std::string& msg);  // sets mi_last_error() (api.cpp)
}

namespace {

// ------------------------------------------------------------------ JSON ---
// A small recursive-descent reader: enough for config.json and safetensors headers.
struct JValue {
  enum Kind { Null, Bool, Number, String, Array, Object } kind = Null;
  bool b = false;
  double num = 0;
  bool is_int = false;
  int64_t i = 0;
  std::string str;
  std::vector<JValue> arr;
  std::vector<std::pair<std::string, JValue>> obj;  // keeps file order

  const JValue* get(const char* key) const {
    if (kind != Object) return nullptr;
    const JValue* hit = nullptr;
    for (auto& kv : obj)
      if (kv.first == key) hit = &kv.second;  // last duplicate wins
    return hit;
  }
};

struct JParser {
  const char* p;
  const char* end;
  std::string err;
  int depth = 0;

  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
  }
  bool fail(const char* what) {
    if (err.empty()) err = what;
    return false;
  }
  bool lit(const char* s) {
    size_t n = strlen(s);
    if ((size_t)(end - p) < n || memcmp(p, s, n)) return false;
    p += n;
    return true;
  }
  static void put_utf8(std::string& o, uint32_t c) {
    if (c < 0x80) {
      o += (char)c;
    } else if (c < 0x800) {
      o += (char)(0xC0 | (c >> 6));
      o += (char)(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      o += (char)(0xE0 | (c >> 12));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    } else {
      o += (char)(0xF0 | (c >> 18));
      o += (char)(0x80 | ((c >> 12) & 0x3F));
      o += (char)(0x80 | ((c >> 6) & 0x3F));
      o += (char)(0x80 | (c & 0x3F));
    }
  }
  bool hex4(uint32_t* out) {
    if (end - p < 4) return fail("truncated \\u escape");
    uint32_t v = 0;
    for (int k = 0; k < 4; ++k) {
      char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else return fail("bad \\u escape");
    }
    *out = v;
    return true;
  }
  bool string(std::string* out) {
    if (p >= end || *p != '"') return fail("expected string");
    ++p;
    out->clear();
    while (p < end && *p != '"') {
      unsigned char c = (unsigned char)*p++;
      if (c < 0x20) return fail("control character in string");
      if (c != '\\') {
        *out += (char)c;
        continue;
      }
      if (p >= end) break;
      char e = *p++;
      switch (e) {
        case '"': *out += '"'; break;
        case '\\': *out += '\\'; break;
        case '/': *out += '/'; break;
        case 'b': *out += '\b'; break;
        case 'f': *out += '\f'; break;
        case 'n': *out += '\n'; break;
        case 'r': *out += '\r'; break;
        case 't': *out += '\t'; break;
        case 'u': {
          uint32_t c1;
          if (!hex4(&c1)) return false;
          if (c1 >= 0xD800 && c1 < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            uint32_t c2;
            if (!hex4(&c2)) return false;
            if (c2 < 0xDC00 || c2 >= 0xE000) return fail("unpaired surrogate");
            c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          } else if (c1 >= 0xD800 && c1 < 0xE000) {
            return fail("unpaired surrogate");
          }
          put_utf8(*out, c1);
          break;
        }
        default: return fail("bad escape");
      }
    }
    if (p >= end) return fail("unterminated string");
    ++p;
    return true;
  }
  bool number(JValue* v) {
    const char* s = p;
    if (p < end && *p == '-') ++p;
    bool frac = false;
    while (p < end && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' ||
                       *p == '+' || *p == '-')) {
      if (*p == '.' || *p == 'e' || *p == 'E') frac = true;
      ++p;
    }
    if (p == s) return fail("expected value");
    std::string t(s, p);
    char* e = nullptr;
    v->kind = JValue::Number;
    v->num = strtod(t.c_str(), &e);
    if (e != t.c_str() + t.size()) return fail("bad number");
    if (!frac) {
      errno = 0;
      long long iv = strtoll(t.c_str(), &e, 10);
      if (errno == 0 && e == t.c_str() + t.size()) {
        v->is_int = true;
        v->i = iv;
      }
    }
    return true;
  }
  bool value(JValue* v) {
    if (++depth > 64) return fail("nesting too deep");
    ws();
    if (p >= end) return fail("unexpected end");
    bool ok = true;
    if (*p == '{') {
      ++p;
      v->kind = JValue::Object;
      ws();
      if (p < end && *p == '}') {
        ++p;
      } else {
        for (;;) {
          ws();
          std::pair<std::string, JValue> kv;
          if (!string(&kv.first)) return false;
          ws();
          if (p >= end || *p != ':') return fail("expected ':'");
          ++p;
          if (!value(&kv.second)) return false;
          v->obj.push_back(std::move(kv));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == '}') { ++p; break; }
          return fail("expected ',' or '}'");
        }
      }
    } else if (*p == '[') {
      ++p;
      v->kind = JValue::Array;
      ws();
      if (p < end && *p == ']') {
        ++p;
      } else {
        for (;;) {
          JValue e;
          if (!value(&e)) return false;
          v->arr.push_back(std::move(e));
          ws();
          if (p < end && *p == ',') { ++p; continue; }
          if (p < end && *p == ']') { ++p; break; }
          return fail("expected ',' or ']'");
        }
      }
    } else if (*p == '"') {
      v->kind = JValue::String;
      ok = string(&v->str);
    } else if (lit("true")) {
      v->kind = JValue::Bool;
      v->b = true;
    } else if (lit("false")) {
      v->kind = JValue::Bool;
    } else if (lit("null")) {
      v->kind = JValue::Null;
    } else {
      ok = number(v);
    }
    --depth;
    return ok;
  }
};

// JSON text must be well-formed UTF-8 (RFC 8259 section 8.1).
bool valid_utf8(const unsigned char* s, size_t n) {
  size_t i = 0;
  while (i < n) {
    unsigned c = s[i];
    int extra;
    uint32_t cp, min;
    if (c < 0x80) { ++i; continue; }
    if ((c & 0xE0) == 0xC0) { extra = 1; cp = c & 0x1F; min = 0x80; }
    else if ((c & 0xF0) == 0xE0) { extra = 2; cp = c & 0x0F; min = 0x800; }
    else if ((c & 0xF8) == 0xF0) { extra = 3; cp = c & 0x07; min = 0x10000; }
    else return false;
    if (n - i <= (size_t)extra) return false;
    for (int k = 1; k <= extra; ++k) {
      if ((s[i + k] & 0xC0) != 0x80) return false;
      cp = (cp << 6) | (s[i + k] & 0x3F);
    }
    if (cp < min || cp > 0x10FFFF || (cp >= 0xD800 && cp < 0xE000)) return false;
    i += extra + 1;
  }
  return true;
}

bool parse_json(const char* s, size_t n, JValue* out, std::string* err) {
  if (!valid_utf8((const unsigned char*)s, n)) {
    *err = "not valid UTF-8";
    return false;
  }
  JParser ps{s, s + n, {}};
  if (!ps.value(out)) {
    *err = ps.err;
    return false;
  }
  ps.ws();
  if (ps.p != ps.end) {
    *err = "trailing characters";
    return false;
  }
  return true;
}

// ---------------------------------------------------------------- dtypes ---
// safetensors dtype strings -> (mlx_dtype code, element bytes). Codes from src/mlx.zig:20-35.
struct DtypeRow {
  const char* name;
  int code;
  int size;
};
constexpr DtypeRow kDtypes[] = {
    {"BOOL", 0, 1}, {"U8", 1, 1},   {"U16", 2, 2},  {"U32", 3, 4},  {"U64", 4, 8},
    {"I8", 5, 1},   {"I16", 6, 2},  {"I32", 7, 4},  {"I64", 8, 8},  {"F16", 9, 2},
    {"F32", 10, 4}, {"F64", 11, 8}, {"BF16", 12, 2}, {"C64", 13, 8},
};

const DtypeRow* find_dtype(const std::string& s) {
  for (auto& r : kDtypes)
    if (s == r.name) return &r;
  return nullptr;
}

bool ends_with(const std::string& s, const char* suf) {
  size_t n = strlen(suf);
  return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}
bool starts_with(const std::string& s, const char* pre) { return s.rfind(pre, 0) == 0; }

// float16 -> float32 (exact), then round-to-nearest-even to bfloat16 (mlx astype).
uint16_t f16_to_bf16(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000) << 16;
  uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF;
  uint32_t f;
  if (exp == 0x1F) {
    f = sign | 0x7F800000u | (man << 13) | (man ? 0x00400000u : 0);
  } else if (exp) {
    f = sign | ((exp + 112) << 23) | (man << 13);
  } else if (man == 0) {
    f = sign;
  } else {  // subnormal: normalise
    int e = -1;
    do {
      man <<= 1;
      ++e;
    } while (!(man & 0x400));
    f = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3FF) << 13);
  }
  if ((f & 0x7F800000u) == 0x7F800000u && (f & 0x7FFFFF)) return (uint16_t)((f >> 16) | 0x40);
  uint32_t r = f + 0x7FFF + ((f >> 16) & 1);
  return (uint16_t)(r >> 16);
}

// ------------------------------------------------------------ the store ---
struct MappedFile {
  std::string path;
  void* base = MAP_FAILED;
  size_t size = 0;
  ~MappedFile() {
    if (base != MAP_FAILED && size) munmap(base, size);
  }
};

struct Tensor {
  std::shared_ptr<MappedFile> file;
  const unsigned char* data = nullptr;
  int64_t raw_bytes = 0;
  int dtype = 0;  // as stored
  int esize = 0;
  bool narrow = false;  // f16 -> bf16 on read
  std::vector<int64_t> shape;
};

bool narrow_1d_enabled() {
  const char* v = getenv("MLX_SERVE_F16_NARROW_1D");
  return !(v && strcmp(v, "0") == 0);
}

// src/model.zig:3148-3185: keys of the vision/audio towers.
bool keep_key(const std::string& k, bool load_vision) {
  static const char* const kVision[] = {"vision_tower.", "embed_vision.", "vision_embedder.",
                                        "embed_audio.", "multi_modal_projector.",
                                        "language_model.multi_modal_projector."};
  static const char* const kAudioTower[] = {"audio_tower.",
                                            "language_model.audio_multi_modal_projector."};
  static const char* const kEncoderVision[] = {"model.encoder.vision_tower.",
                                               "model.encoder.embed_vision."};
  static const char* const kNestedVision[] = {"model.vision_tower.", "model.vision_adapter.",
                                              "model.vision_projection.", "vision_adapter.",
                                              "vision_projection.", "model.visual."};
  for (auto pre : kAudioTower)
    if (starts_with(k, pre)) return false;
  for (auto pre : kEncoderVision)
    if (starts_with(k, pre)) return false;
  if (!load_vision) {
    for (auto pre : kNestedVision)
      if (starts_with(k, pre)) return false;
    for (auto pre : kVision)
      if (starts_with(k, pre)) return false;
  }
  return true;
}

}  // namespace

struct mi_ckpt {
  mi_quant_config quant{0, 64, MI_QMODE_AFFINE};
  std::map<std::string, Tensor> tensors;
  std::vector<const std::string*> names;  // sorted view for mi_ckpt_name
  bool narrow_1d = true;

  void index_names() {
    names.clear();
    for (auto& kv : tensors) names.push_back(&kv.first);
  }
};

namespace {

int err(int code, const std::string& m) { return mi::report_error(code, m); }

int load_file(mi_ckpt* ck, const std::string& path, bool load_vision) {
  auto mf = std::make_shared<MappedFile>();
  mf->path = path;
  int fd = open(path.c_str(), O_RDONLY);
  if (fd < 0) return err(MI_ERR_INVALID, path + ": cannot open: " + strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return err(MI_ERR_INVALID, path + ": cannot stat");
  }
  mf->size = (size_t)st.st_size;
  if (mf->size < 8) {
    close(fd);
    return err(MI_ERR_INVALID, path + ": too short for a safetensors header");
  }
  mf->base = mmap(nullptr, mf->size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (mf->base == MAP_FAILED) return err(MI_ERR_INVALID, path + ": mmap failed");
  const unsigned char* b = (const unsigned char*)mf->base;
  uint64_t hlen = 0;
  for (int k = 7; k >= 0; --k) hlen = (hlen << 8) | b[k];
  if (hlen > mf->size - 8) return err(MI_ERR_INVALID, path + ": header length past end of file");
  JValue hdr;
  std::string perr;
  if (!parse_json((const char*)b + 8, (size_t)hlen, &hdr, &perr))
    return err(MI_ERR_INVALID, path + ": bad header JSON: " + perr);
  if (hdr.kind != JValue::Object) return err(MI_ERR_INVALID, path + ": header is not an object");
  const unsigned char* data = b + 8 + hlen;
  uint64_t data_len = mf->size - 8 - hlen;
  std::vector<std::pair<std::string, Tensor>> found;
  for (auto& kv : hdr.obj) {
    if (kv.first == "__metadata__") continue;
    const JValue& t = kv.second;
    const JValue* dt = t.get("dtype");
    const JValue* sh = t.get("shape");
    const JValue* off = t.get("data_offsets");
    if (!dt || dt->kind != JValue::String || !sh || sh->kind != JValue::Array || !off ||
        off->kind != JValue::Array || off->arr.size() != 2)
      return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' lacks dtype/shape/data_offsets");
    const DtypeRow* row = find_dtype(dt->str);
    if (!row) return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' has dtype " + dt->str);
    if (sh->arr.size() > MI_CKPT_MAX_DIMS)
      return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' has too many dims");
    Tensor ten;
    ten.file = mf;
    ten.dtype = row->code;
    ten.esize = row->size;
    uint64_t elems = 1;
    for (auto& d : sh->arr) {
      if (d.kind != JValue::Number || !d.is_int || d.i < 0)
        return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' has a bad shape");
      ten.shape.push_back(d.i);
      if (d.i && elems > (UINT64_MAX / 16) / (uint64_t)d.i)
        return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' is too large");
      elems *= (uint64_t)d.i;
    }
    const JValue &o0 = off->arr[0], &o1 = off->arr[1];
    if (o0.kind != JValue::Number || !o0.is_int || o1.kind != JValue::Number || !o1.is_int ||
        o0.i < 0 || o1.i < o0.i || (uint64_t)o1.i > data_len)
      return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' has data_offsets out of range");
    if ((uint64_t)(o1.i - o0.i) != elems * (uint64_t)row->size)
      return err(MI_ERR_INVALID, path + ": tensor '" + kv.first + "' byte size does not match its shape");
    ten.data = data + o0.i;
    ten.raw_bytes = o1.i - o0.i;
    ten.narrow = row->code == MI_DTYPE_FLOAT16 &&
                 (ends_with(kv.first, ".scales") || ends_with(kv.first, ".biases") ||
                  (ten.shape.size() == 1 && ck->narrow_1d));
    if (!keep_key(kv.first, load_vision)) continue;
    found.emplace_back(kv.first, std::move(ten));
  }
  for (auto& f : found) ck->tensors[f.first] = std::move(f.second);  // later file wins
  return MI_OK;
}

const Tensor* lookup(const mi_ckpt* ck, const std::string& name) {
  auto it = ck->tensors.find(name);
  return it == ck->tensors.end() ? nullptr : &it->second;
}

int64_t last_dim(const Tensor& t) { return t.shape.size() >= 2 ? t.shape.back() : 0; }

// fpQuantModeFor (src/transformer.zig:16850-16855).
int fp_mode_for(int64_t bits, int64_t gs) {
  if (bits == 8 && gs == 32) return MI_QMODE_MXFP8;
  if (bits == 4 && gs == 32) return MI_QMODE_MXFP4;
  if (bits == 4 && gs == 16) return MI_QMODE_NVFP4;
  return -1;
}

}  // namespace

extern "C" {

int mi_parse_quant_config(const char* json, size_t len, mi_quant_config* out) {
  if (!json || !out) return err(MI_ERR_INVALID, "null argument");
  JValue root;
  std::string perr;
  if (!parse_json(json, len, &root, &perr)) return err(MI_ERR_INVALID, "config.json: " + perr);
  if (root.kind != JValue::Object) return err(MI_ERR_INVALID, "config.json is not an object");
  mi_quant_config q{0, 64, MI_QMODE_AFFINE};
  if (const JValue* qv = root.get("quantization")) {
    if (qv->kind != JValue::Object) return err(MI_ERR_INVALID, "\"quantization\" is not an object");
    if (const JValue* v = qv->get("bits")) {
      if (v->kind != JValue::Number || !v->is_int || v->i < 0 || v->i > 64)
        return err(MI_ERR_INVALID, "quantization.bits is not a small integer");
      q.bits = (int)v->i;
    }
    if (const JValue* v = qv->get("group_size")) {
      if (v->kind != JValue::Number || !v->is_int || v->i <= 0 || v->i > (1 << 20))
        return err(MI_ERR_INVALID, "quantization.group_size is not a positive integer");
      q.group_size = (int)v->i;
    }
    if (const JValue* v = qv->get("mode")) {
      if (v->kind == JValue::String) {
        static const char* const kModes[] = {"affine", "nvfp4", "mxfp4", "mxfp8"};
        int m = -1;
        for (int k = 0; k < 4; ++k)
          if (v->str == kModes[k]) m = k;
        if (m < 0)
          return err(MI_ERR_INVALID, "unsupported quantization mode '" + v->str +
                                         "' (supported: affine, nvfp4, mxfp4, mxfp8)");
        q.mode = m;
      }
    }
    if (q.mode == MI_QMODE_AFFINE && q.bits != 0) {
      switch (q.bits) {
        case 2: case 3: case 4: case 5: case 6: case 8: break;
        default:
          return err(MI_ERR_INVALID, "unsupported affine quantization: " + std::to_string(q.bits) +
                                         "-bit (supported: 2, 3, 4, 5, 6, 8)");
      }
    }
  }
  *out = q;
  return MI_OK;
}

int mi_ckpt_open(const char* model_dir, int load_vision, mi_ckpt** out) {
  if (!model_dir || !out) return err(MI_ERR_INVALID, "null argument");
  *out = nullptr;
  std::unique_ptr<mi_ckpt> ck(new mi_ckpt);
  ck->narrow_1d = narrow_1d_enabled();
  std::string dir = model_dir;
  DIR* d = opendir(model_dir);
  if (!d) return err(MI_ERR_INVALID, dir + ": cannot open directory");
  std::vector<std::string> files;
  bool have_config = false;
  while (struct dirent* e = readdir(d)) {
    std::string n = e->d_name;
    if (n == "config.json") have_config = true;
    if (!ends_with(n, ".safetensors")) continue;
    struct stat st;
    std::string full = dir + "/" + n;
    if (stat(full.c_str(), &st) == 0 && S_ISREG(st.st_mode)) files.push_back(n);  // follows symlinks
  }
  closedir(d);
  std::sort(files.begin(), files.end());
  if (have_config) {
    std::string full = dir + "/config.json";
    FILE* f = fopen(full.c_str(), "rb");
    if (!f) return err(MI_ERR_INVALID, full + ": cannot open");
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof buf, f)) > 0) text.append(buf, n);
    fclose(f);
    int rc = mi_parse_quant_config(text.data(), text.size(), &ck->quant);
    if (rc) return rc;
  }
  for (auto& n : files) {
    int rc = load_file(ck.get(), dir + "/" + n, load_vision != 0);
    if (rc) return rc;
  }
  if (ck->tensors.empty())
    return err(MI_ERR_INVALID, "no usable weights loaded from " + dir + " (" +
                                   std::to_string(files.size()) +
                                   " *.safetensors file(s) found): incomplete checkpoint");
  ck->index_names();
  *out = ck.release();
  return MI_OK;
}

int mi_ckpt_open_file(const char* path, mi_ckpt** out) {
  if (!path || !out) return err(MI_ERR_INVALID, "null argument");
  *out = nullptr;
  std::unique_ptr<mi_ckpt> ck(new mi_ckpt);
  ck->narrow_1d = narrow_1d_enabled();
  int rc = load_file(ck.get(), path, false);
  if (rc) return rc;
  if (ck->tensors.empty())
    return err(MI_ERR_INVALID, std::string("no usable weights loaded from ") + path);
  ck->index_names();
  *out = ck.release();
  return MI_OK;
}

void mi_ckpt_close(mi_ckpt* ck) { delete ck; }

int mi_ckpt_quant_config(const mi_ckpt* ck, mi_quant_config* out) {
  if (!ck || !out) return err(MI_ERR_INVALID, "null argument");
  *out = ck->quant;
  return MI_OK;
}

int mi_ckpt_set_quant_config(mi_ckpt* ck, const mi_quant_config* cfg) {
  if (!ck || !cfg) return err(MI_ERR_INVALID, "null argument");
  if (cfg->mode < MI_QMODE_AFFINE || cfg->mode > MI_QMODE_MXFP8 || cfg->bits < 0 ||
      cfg->group_size <= 0)
    return err(MI_ERR_INVALID, "bad quantization config");
  ck->quant = *cfg;
  return MI_OK;
}

int64_t mi_ckpt_count(const mi_ckpt* ck) { return ck ? (int64_t)ck->names.size() : 0; }

const char* mi_ckpt_name(const mi_ckpt* ck, int64_t i) {
  if (!ck || i < 0 || i >= (int64_t)ck->names.size()) return nullptr;
  return ck->names[(size_t)i]->c_str();
}

int mi_ckpt_info(const mi_ckpt* ck, const char* name, mi_tensor_info* info) {
  if (!ck || !name || !info) return err(MI_ERR_INVALID, "null argument");
  const Tensor* t = lookup(ck, name);
  if (!t) return err(MI_ERR_INVALID, std::string("MISSING WEIGHT: ") + name);
  memset(info, 0, sizeof *info);
  info->dtype = t->narrow ? MI_DTYPE_BFLOAT16 : t->dtype;
  info->ndim = (int)t->shape.size();
  for (size_t k = 0; k < t->shape.size(); ++k) info->shape[k] = t->shape[k];
  info->nbytes = t->raw_bytes;  // f16 and bf16 are both 2 bytes
  return MI_OK;
}

int mi_ckpt_read(const mi_ckpt* ck, const char* name, void* dst, size_t bytes) {
  if (!ck || !name || (!dst && bytes)) return err(MI_ERR_INVALID, "null argument");
  const Tensor* t = lookup(ck, name);
  if (!t) return err(MI_ERR_INVALID, std::string("MISSING WEIGHT: ") + name);
  if (bytes < (size_t)t->raw_bytes)
    return err(MI_ERR_INVALID, std::string(name) + ": destination holds " + std::to_string(bytes) +
                                   " bytes, tensor needs " + std::to_string(t->raw_bytes));
  if (!t->narrow) {
    memcpy(dst, t->data, (size_t)t->raw_bytes);
  } else {
    const unsigned char* s = t->data;
    uint16_t* o = (uint16_t*)dst;
    for (int64_t k = 0; k < t->raw_bytes / 2; ++k) o[k] = f16_to_bf16((uint16_t)(s[2 * k] | (s[2 * k + 1] << 8)));
  }
  return MI_OK;
}

int mi_ckpt_upload(const mi_ckpt* ck, const char* name, void* dst, size_t bytes) {
  if (!ck || !name || (!dst && bytes)) return err(MI_ERR_INVALID, "null argument");
  const Tensor* t = lookup(ck, name);
  if (!t) return err(MI_ERR_INVALID, std::string("MISSING WEIGHT: ") + name);
  if (bytes < (size_t)t->raw_bytes)
    return err(MI_ERR_INVALID, std::string(name) + ": destination too small");
  if (!t->raw_bytes) return MI_OK;
  const void* src = t->data;
  std::vector<unsigned char> staged;
  if (t->narrow) {
    staged.resize((size_t)t->raw_bytes);
    int rc = mi_ckpt_read(ck, name, staged.data(), staged.size());
    if (rc) return rc;
    src = staged.data();
  }
  hipError_t e = hipMemcpy(dst, src, (size_t)t->raw_bytes, hipMemcpyHostToDevice);
  if (e != hipSuccess)
    return err(MI_ERR_HIP, std::string("hipMemcpy(") + name + "): " + hipGetErrorString(e));
  return MI_OK;
}

int mi_ckpt_linear(const mi_ckpt* ck, const char* prefix, int64_t in_dim, mi_linear_desc* out) {
  if (!ck || !prefix || !out || in_dim < 0) return err(MI_ERR_INVALID, "bad argument");
  std::string p = prefix;
  const Tensor* w = lookup(ck, p + ".weight");
  if (!w) return err(MI_ERR_INVALID, "MISSING WEIGHT: " + p + ".weight");
  if (w->shape.size() < 2) return err(MI_ERR_INVALID, p + ".weight is not a matrix");
  mi_linear_desc d{};
  d.out_dim = w->shape[w->shape.size() - 2];
  const mi_quant_config& q = ck->quant;
  if (q.bits == 0) {  // dense checkpoint: scales/biases are empty placeholders
    d.bits = 0;
    d.group_size = q.group_size;
    d.mode = MI_QMODE_AFFINE;
    d.in_dim = w->shape.back();
    *out = d;
    return MI_OK;
  }
  const Tensor* s = lookup(ck, p + ".scales");
  if (!s) return err(MI_ERR_INVALID, "MISSING WEIGHT: " + p + ".scales");
  const Tensor* b = lookup(ck, p + ".biases");
  if (!b && q.mode == MI_QMODE_AFFINE) return err(MI_ERR_INVALID, "MISSING WEIGHT: " + p + ".biases");
  d.has_scales = 1;
  d.has_biases = b != nullptr;

  // computeQuantParams.
  const int64_t w_cols = last_dim(*w), s_cols = last_dim(*s);
  if (s->dtype == MI_DTYPE_UINT8) {
    if (q.mode != MI_QMODE_AFFINE) {
      d.bits = q.bits;
      d.group_size = q.group_size;
      d.mode = q.mode;
      if (in_dim > 0 && w_cols > 0 && s_cols > 0 && (w_cols * 32) % in_dim == 0 &&
          in_dim % s_cols == 0) {
        int64_t bits = w_cols * 32 / in_dim, gs = in_dim / s_cols;
        int m = fp_mode_for(bits, gs);
        if (!(bits == q.bits && gs == q.group_size) && m >= 0) {
          d.bits = (int)bits;
          d.group_size = (int)gs;
          d.mode = m;
        }
      }
    } else {  // an mxfp8 tensor inside an affine checkpoint
      d.bits = 8;
      d.group_size = (w_cols > 0 && s_cols > 0) ? (int)((w_cols * 32) / (s_cols * 8)) : 32;
      d.mode = MI_QMODE_MXFP8;
    }
  } else if (q.mode == MI_QMODE_AFFINE) {
    int bits = 0, gs = 0;
    if (in_dim > 0 && mi_affine_params_from_geometry(w_cols, s_cols, in_dim, &bits, &gs) == MI_OK) {
      d.bits = bits;
      d.group_size = gs;
    } else {  // detectQuantBits against the declared group size
      d.bits = (w->shape.size() < 2 || s->shape.size() < 2 || s_cols == 0)
                   ? 4
                   : (int)((w_cols * 32) / (s_cols * q.group_size));
      d.group_size = q.group_size;
    }
    d.mode = MI_QMODE_AFFINE;
  } else {  // affine override inside an fp checkpoint
    d.mode = MI_QMODE_AFFINE;
    if (in_dim > 0 && s_cols > 0 && w_cols > 0) {
      d.bits = (int)((w_cols * 32) / in_dim);
      d.group_size = (int)(in_dim / s_cols);
    } else if (w_cols > 0 && s_cols > 0) {
      d.bits = std::max<int>((int)((w_cols * 32) / s_cols) / 64, 1);
      d.group_size = 64;
    } else {
      d.bits = 8;
      d.group_size = 64;
    }
  }
  d.in_dim = in_dim > 0 ? in_dim : (d.bits > 0 ? w_cols * 32 / d.bits : 0);
  *out = d;
  return MI_OK;
}

}  // extern "C"
