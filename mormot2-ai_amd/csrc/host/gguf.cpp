// gguf.cpp - GGUF v3 files: a validated, memory-mapped reader (TGgufFile,
// src/infer/mormot.ai.infer.loader.gguf.pas) and the decoder description of a
// llama.cpp file of the qwen3, qwen3moe and gpt-oss architectures
// (TQwen3Model / TQwen3MoeModel / TGptOssModel.LoadGgufConfig and LoadWeights,
// model.qwen3.pas:405-620, :797-846, model.gptoss.pas:321-475, :700-760).
//
// The format (ggml docs/gguf.md): magic "GGUF", version 3, tensor and
// key/value counts, the key/value pairs, the tensor infos (name, dimensions
// innermost first, ggml type, offset), padding to the alignment, the data.
// Every read is bounded by the file size and every count is checked against
// what the remaining bytes can hold before anything is allocated; the checks
// are those of TGgufFile.Parse (loader.gguf.pas:405-585), with the same
// reasons in the error text. Shapes are reported row-major: [ne1, ne0].
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdlib>
#include <strings.h>
#include <initializer_list>
#include <cmath>
#include <cstring>
#include <map>
#include <memory>

#include "internal.h"

using namespace ihip;

namespace {

enum : int32_t { U8, I8, U16, I16, U32, I32, F32V, BOOLV, STR, ARR, U64, I64, F64V, NTYPES };
const char* const TYPE_NAME[NTYPES] = {"UINT8", "INT8", "UINT16", "INT16", "UINT32", "INT32", "FLOAT32",
                                      "BOOL", "STRING", "ARRAY", "UINT64", "INT64", "FLOAT64"};
const int TYPE_SIZE[NTYPES] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
constexpr int64_t DEFAULT_ALIGNMENT = 32, MAX_DIMS = 4, MAX_ITEMS = int64_t(1) << 24;

// the ggml type ids this path reads, as TInferDType ordinals (GgufTensorType,
// loader.gguf.pas:206-232)
int dtype_of_ggml(uint32_t t)
{
  switch (t) {
    case 0: return DT_F32;
    case 1: return DT_F16;
    case 2: return DT_Q4_0;
    case 6: return DT_Q5_0;
    case 7: return DT_Q5_1;
    case 8: return DT_Q8_0;
    case 12: return DT_Q4_K;
    case 14: return DT_Q6_K;
    case 30: return DT_BF16;
    case 39: return DT_MXFP4;
    default: return 0;
  }
}

const char* ggml_name(uint32_t t)
{
  static const char* const n[] = {"F32",     "F16",    "Q4_0",    "Q4_1",   "?",      "?",      "Q5_0",
                                  "Q5_1",    "Q8_0",   "Q8_1",    "Q2_K",   "Q3_K",   "Q4_K",   "Q5_K",
                                  "Q6_K",    "Q8_K",   "IQ2_XXS", "IQ2_XS", "IQ3_XXS", "IQ1_S", "IQ4_NL",
                                  "IQ3_S",   "IQ2_S",  "IQ4_XS",  "I8",     "I16",    "I32",    "I64",
                                  "F64",     "IQ1_M",  "BF16"};
  if (t < sizeof n / sizeof n[0]) return n[t];
  if (t == 34) return "TQ1_0";
  if (t == 35) return "TQ2_0";
  if (t == 39) return "MXFP4";
  return "?";
}

const char* dtype_name(int dt)
{
  switch (dt) {
    case DT_F32: return "F32";
    case DT_F16: return "F16";
    case DT_BF16: return "BF16";
    case DT_Q8_0: return "Q8_0";
    case DT_Q4_0: return "Q4_0";
    case DT_Q4_K: return "Q4_K";
    case DT_Q6_K: return "Q6_K";
    case DT_Q5_0: return "Q5_0";
    case DT_MXFP4: return "MXFP4";
    case DT_Q5_1: return "Q5_1";
    default: return "?";
  }
}

bool block_type(int dt) { return dt != DT_F32 && dt != DT_F16 && dt != DT_BF16; }

struct Value {
  std::string key;
  int32_t vtype, etype;
  int64_t count;
  const uint8_t* data;  // the value, or the first element (a string: its 8-byte length first)
  std::vector<const uint8_t*> strings;  // a string array: where each element starts
};

struct Tensor {
  std::string name;
  int32_t dtype, ndim;
  int64_t shape[4];  // row-major
  int64_t count, bytes, off;
  const uint8_t* data;
};

// a format error: the message goes to ihip_last_error()
struct Refused {
  std::string msg;
};

std::string fmt(const char* f, ...) __attribute__((format(printf, 1, 2)));
std::string fmt(const char* f, ...)
{
  char b[512];
  va_list ap;
  va_start(ap, f);
  vsnprintf(b, sizeof b, f, ap);
  va_end(ap);
  return b;
}

}  // namespace

struct ihip_gguf {
  std::string name;  // the file name, or "content" for a copied buffer
  const uint8_t* buf = nullptr;
  int64_t size = 0;
  void* map = nullptr;
  std::vector<uint8_t> own;
  std::vector<Value> values;
  std::map<std::string, int64_t> keys;
  std::vector<Tensor> tensors;
  std::map<std::string, int64_t> names;
  int64_t alignment = DEFAULT_ALIGNMENT, data_start = 0;
  // the decoder description (ihip_gguf_model_desc): norms widened to F32
  std::vector<std::unique_ptr<std::vector<float>>> widened;
  std::vector<ihip_layer_desc> layers;
  ihip_model_desc desc{};
  bool have_desc = false;

  [[noreturn]] void refuse(const std::string& m) const { throw Refused{"GGUF " + name + ": " + m}; }
  void parse();
  const Value* find(const std::string& k) const
  {
    auto it = keys.find(k);
    return it == keys.end() ? nullptr : &values[it->second];
  }
  const Value& value(const std::string& k, int32_t type) const
  {
    const Value* v = find(k);
    if (!v) refuse("no metadata " + k);
    if (v->vtype != type) refuse(k + " is " + TYPE_NAME[v->vtype] + ", expected " + TYPE_NAME[type]);
    return *v;
  }
  std::string str(const std::string& k) const
  {
    const Value& v = value(k, STR);
    int64_t n;
    memcpy(&n, v.data, 8);
    return std::string((const char*)v.data + 8, (size_t)n);
  }
  int64_t integer(const std::string& k) const
  {
    const Value* v = find(k);
    if (!v) refuse("no metadata " + k);
    const uint8_t* p = v->data;
    switch (v->vtype) {
      case U8: return *p;
      case I8: return (int8_t)*p;
      case U16: { uint16_t x; memcpy(&x, p, 2); return x; }
      case I16: { int16_t x; memcpy(&x, p, 2); return x; }
      case U32: { uint32_t x; memcpy(&x, p, 4); return x; }
      case I32: { int32_t x; memcpy(&x, p, 4); return x; }
      case U64:
      case I64: {
        int64_t x;
        memcpy(&x, p, 8);
        if (v->vtype == U64 && x < 0) refuse(k + " is out of range");
        return x;
      }
      default: refuse(k + " is " + TYPE_NAME[v->vtype] + ", expected an integer");
    }
  }
  double real(const std::string& k) const
  {
    const Value* v = find(k);
    if (!v) refuse("no metadata " + k);
    if (v->vtype == F32V) { float x; memcpy(&x, v->data, 4); return x; }
    if (v->vtype == F64V) { double x; memcpy(&x, v->data, 8); return x; }
    refuse(k + " is " + TYPE_NAME[v->vtype] + ", expected a float");
  }
  bool boolean(const std::string& k) const { return *value(k, BOOLV).data != 0; }
  const Value& array(const std::string& k, int32_t elem, int64_t count) const
  {
    const Value& v = value(k, ARR);
    if (v.etype != elem)
      refuse(k + " is an array of " + TYPE_NAME[v.etype] + ", expected " + TYPE_NAME[elem]);
    if (count >= 0 && v.count != count)
      refuse(fmt("%s has %lld elements, expected %lld", k.c_str(), (long long)v.count, (long long)count));
    return v;
  }
  const Tensor* tensor(const std::string& n) const
  {
    auto it = names.find(n);
    return it == names.end() ? nullptr : &tensors[it->second];
  }
};

namespace {

// a bounded cursor over the header (TGgufReader, loader.gguf.pas:236-300)
struct Reader {
  const ihip_gguf* g;
  const uint8_t *start, *cur;
  int64_t left;
  void need(int64_t n, const std::string& what) const
  {
    if (n < 0 || n > left) g->refuse(what + " runs past the end of the file");
  }
  uint32_t u32(const std::string& what)
  {
    need(4, what);
    uint32_t v;
    memcpy(&v, cur, 4);
    cur += 4;
    left -= 4;
    return v;
  }
  int64_t u64(const std::string& what)
  {
    need(8, what);
    int64_t v;
    memcpy(&v, cur, 8);
    cur += 8;
    left -= 8;
    // a count or length above the int64 range can never fit the file
    if (v < 0) g->refuse(what + " is out of range");
    return v;
  }
  void skip(int64_t n, const std::string& what)
  {
    need(n, what);
    cur += n;
    left -= n;
  }
  std::string str(const std::string& what)
  {
    int64_t n = u64(what);
    need(n, what);
    if (memchr(cur, 0, (size_t)n)) g->refuse(what + " contains NUL");
    std::string s((const char*)cur, (size_t)n);
    cur += n;
    left -= n;
    return s;
  }
  int64_t pos() const { return cur - start; }
};

}  // namespace

void ihip_gguf::parse()
{
  Reader r{this, buf, buf, size};
  if (r.u32("magic") != 0x46554747u) refuse("not a GGUF file");
  const uint32_t version = r.u32("version");
  if (version != 3) refuse(fmt("GGUF version %u not supported (only 3)", version));
  const int64_t nt = r.u64("tensor count"), nv = r.u64("key/value count");
  // a key/value pair takes at least 12 bytes, a tensor info at least 32: a
  // hostile count is refused before any allocation
  if (nt > r.left / 32 || nv > r.left / 12 || nt > MAX_ITEMS || nv > MAX_ITEMS)
    refuse(fmt("%lld tensors and %lld values cannot fit %lld bytes", (long long)nt, (long long)nv,
               (long long)size));
  auto scalar = [&](int32_t t, const std::string& what) {
    if (t == STR) {
      int64_t n = r.u64(what);
      r.need(n, what);
      if (memchr(r.cur, 0, (size_t)n)) refuse(what + " contains NUL");
      r.skip(n, what);
    } else if (t == BOOLV) {
      r.need(1, what);
      if (*r.cur > 1) refuse(fmt("%s is a BOOL of value %u", what.c_str(), *r.cur));
      r.skip(1, what);
    } else {
      r.skip(TYPE_SIZE[t], what);
    }
  };
  values.resize((size_t)nv);
  for (int64_t i = 0; i < nv; i++) {
    Value& v = values[i];
    v.key = r.str("a key");
    if (v.key.empty()) refuse("empty key");
    uint32_t t = r.u32(v.key);
    if (t >= NTYPES) refuse(fmt("%s has unknown type %u", v.key.c_str(), t));
    v.vtype = v.etype = (int32_t)t;
    v.count = 1;
    if (t == ARR) {
      uint32_t e = r.u32(v.key);
      if (e >= NTYPES) refuse(fmt("%s has unknown element type %u", v.key.c_str(), e));
      v.etype = (int32_t)e;
      if (e == ARR) refuse(v.key + " is a nested array");
      v.count = r.u64(v.key);
      v.data = r.cur;
      // every element takes at least one byte, a string at least 8
      if (v.count > r.left || (e == STR && v.count > r.left / 8))
        refuse(fmt("%s has %lld elements - more than the file holds", v.key.c_str(), (long long)v.count));
      if (e == STR || e == BOOLV) {
        if (e == STR) v.strings.reserve((size_t)v.count);
        for (int64_t j = 0; j < v.count; j++) {
          if (e == STR) v.strings.push_back(r.cur);
          scalar((int32_t)e, v.key);
        }
      } else {
        if (v.count > r.left / TYPE_SIZE[e])
          refuse(fmt("%s has %lld elements - more than the file holds", v.key.c_str(), (long long)v.count));
        r.skip(v.count * TYPE_SIZE[e], v.key);
      }
    } else {
      v.data = r.cur;
      scalar((int32_t)t, v.key);
    }
    if (!keys.emplace(v.key, i).second) refuse("key \"" + v.key + "\" defined twice");
  }
  // the alignment of the data section
  alignment = DEFAULT_ALIGNMENT;
  if (const Value* a = find("general.alignment")) {
    if (a->vtype != U32) refuse(std::string("general.alignment is ") + TYPE_NAME[a->vtype] + " instead of UINT32");
    uint32_t x;
    memcpy(&x, a->data, 4);
    alignment = x;
    if (alignment == 0 || (alignment & (alignment - 1)))
      refuse(fmt("alignment %lld is no power of two", (long long)alignment));
  }
  // tensor infos
  tensors.resize((size_t)nt);
  for (int64_t i = 0; i < nt; i++) {
    Tensor& ti = tensors[i];
    ti.name = r.str("a tensor name");
    if (ti.name.empty()) refuse("tensor without a name");
    const uint32_t nd = r.u32(ti.name);
    if (nd == 0 || nd > MAX_DIMS) refuse(fmt("%s has %u dimensions", ti.name.c_str(), nd));
    int64_t ne[4];
    for (uint32_t j = 0; j < nd; j++) ne[j] = r.u64(ti.name);
    const uint32_t t = r.u32(ti.name);
    ti.dtype = dtype_of_ggml(t);
    if (!ti.dtype) refuse(fmt("%s has unsupported ggml type %u (%s)", ti.name.c_str(), t, ggml_name(t)));
    const int64_t off = r.u64(ti.name);
    ti.ndim = (int32_t)nd;
    // row-major: innermost dimension last
    for (uint32_t j = 0; j < nd; j++) {
      const int64_t d = ne[nd - 1 - j];
      if (d <= 0) refuse(fmt("%s has a dimension of %lld", ti.name.c_str(), (long long)d));
      ti.shape[j] = d;
    }
    for (uint32_t j = nd; j < 4; j++) ti.shape[j] = 1;
    // a block type packs whole blocks per row
    const int bv = block_values(ti.dtype), bb = block_bytes(ti.dtype);
    if (ne[0] % bv)
      refuse(fmt("%s rows of %lld are no whole %s blocks", ti.name.c_str(), (long long)ne[0],
                 dtype_name(ti.dtype)));
    // the element count and byte size, each step bounded by the file size
    // at most 2 values per byte of the file (every type packs fewer): the
    // products cannot overflow; the range itself is checked below
    const int64_t limit = 2 * size;
    int64_t count = 1;
    bool fits = true;
    for (uint32_t j = 0; j < nd && fits; j++) {
      if (ne[j] > limit || count > limit / ne[j]) fits = false;
      else count *= ne[j];
    }
    if (!fits) refuse(ti.name + " shape exceeds the file");
    ti.count = count;
    ti.bytes = count / bv * bb;
    ti.off = off;
    if (off % alignment) refuse(fmt("%s offset %lld is not aligned to %lld", ti.name.c_str(), (long long)off,
                                    (long long)alignment));
    if (off > size) refuse(fmt("%s offset %lld outside the file", ti.name.c_str(), (long long)off));
    if (!names.emplace(ti.name, i).second) refuse("tensor \"" + ti.name + "\" defined twice");
  }
  // the data section starts at the next multiple of the alignment
  data_start = r.pos();
  if (data_start % alignment) data_start += alignment - data_start % alignment;
  if (data_start > size) refuse("no data section");
  const int64_t data_len = size - data_start;
  // tensors follow each other in file order: each at the aligned end of the
  // one before; after the last, at most the padding
  int64_t prev_end = 0;
  for (Tensor& ti : tensors) {
    int64_t n = prev_end;
    if (n % alignment) n += alignment - n % alignment;
    if (ti.off != n)
      refuse(fmt("%s starts at %lld, expected %lld (overlap, gap or order)", ti.name.c_str(), (long long)ti.off,
                 (long long)n));
    if (ti.bytes > data_len - ti.off)
      refuse(fmt("%s range [%lld,%lld) outside the %lld data bytes", ti.name.c_str(), (long long)ti.off,
                 (long long)(ti.off + ti.bytes), (long long)data_len));
    ti.data = buf + data_start + ti.off;
    prev_end = ti.off + ti.bytes;
  }
  if (data_len - prev_end >= alignment)
    refuse(fmt("%lld unreferenced bytes after the last tensor", (long long)(data_len - prev_end)));
}

// ------------------------------------------------------------ the decoder
namespace {

struct DescBuilder {
  ihip_gguf* g;
  std::string arch;
  int used = 0;    // tensors understood
  int trunk = -1;  // the tensors of the model (-1: every tensor of the file)

  [[noreturn]] void refuse(const std::string& m) const { g->refuse(m); }
  // a count of the metadata, bounded (GgufCount, model.qwen3.pas:405-413)
  int32_t count(const std::string& key) const
  {
    int64_t v = g->integer(arch + "." + key);
    if (v <= 0 || v > (int64_t(1) << 30))
      refuse(fmt("%s.%s = %lld out of range", arch.c_str(), key.c_str(), (long long)v));
    return (int32_t)v;
  }
  bool has(const std::string& key) const { return g->find(arch + "." + key) != nullptr; }
  // the tensor, its row-major shape and type checked (TDecoderModel.Checked,
  // decoder.pas:1922-1960): F32/BF16/F16, and the block types for a matrix
  const Tensor& checked(const std::string& name, std::initializer_list<int64_t> dims, bool blocks) const
  {
    const Tensor* t = g->tensor(name);
    if (!t) refuse("no tensor " + name + " in " + g->name);
    bool ok = t->ndim == (int)dims.size();
    int j = 0;
    for (int64_t d : dims) ok = ok && t->shape[j++] == d;
    if (!ok) {
      std::string have, want;
      for (int i = 0; i < t->ndim; i++) have += (i ? "," : "") + std::to_string(t->shape[i]);
      j = 0;
      for (int64_t d : dims) want += (j++ ? "," : "") + std::to_string(d);
      refuse(name + " is shaped [" + have + "], expected [" + want + "]");
    }
    if (block_type(t->dtype) && !blocks)
      refuse(name + " is " + dtype_name(t->dtype) + ", not supported here");
    return *t;
  }
  // every fp16 scale of a block tensor finite; MXFP4 exponents inside the
  // range computed exactly unless the block is all zeros (CheckScales,
  // CheckMxfp4Scales, decoder.pas:2118-2167)
  void check_scales(const Tensor& t, const std::string& name) const
  {
    const int bb = block_bytes(t.dtype);
    const int64_t nb = t.count / block_values(t.dtype);
    const uint8_t* p = t.data;
    if (t.dtype == DT_MXFP4) {
      for (int64_t b = 0; b < nb; b++, p += bb) {
        const uint8_t e = p[0];
        if (e < 104 || e > 143)
          for (int j = 0; j < 16; j++)
            if (p[1 + j] & 0x77)
              refuse(fmt("%s has the MXFP4 exponent %u in block %lld, beyond the range computed exactly",
                         name.c_str(), e, (long long)b));
      }
      return;
    }
    int first = 0, second = -1;
    if (t.dtype == DT_Q4_K || t.dtype == DT_Q5_1) second = 2;
    if (t.dtype == DT_Q6_K) first = bb - 2;
    for (int64_t b = 0; b < nb; b++, p += bb) {
      uint16_t a, c = 0;
      memcpy(&a, p + first, 2);
      if (second >= 0) memcpy(&c, p + second, 2);
      if ((a & 0x7fff) >= 0x7c00 || (second >= 0 && (c & 0x7fff) >= 0x7c00))
        refuse(fmt("%s has a scale that is no finite number in block %lld", name.c_str(), (long long)b));
    }
  }
  // a vector or small tensor as F32: in place, or BF16/F16 widened exactly
  // (TDecoderModel.Weight / WidenTensor, decoder.pas:1962-2000)
  ihip_tensor weight(const std::string& name, std::initializer_list<int64_t> dims)
  {
    const Tensor& t = checked(name, dims, false);
    used++;
    if (t.dtype == DT_F32) return ihip_tensor{t.data, DT_F32, 0};
    auto v = std::make_unique<std::vector<float>>((size_t)t.count);
    const uint16_t* s = (const uint16_t*)t.data;
    for (int64_t i = 0; i < t.count; i++) {
      uint16_t h;
      memcpy(&h, s + i, 2);
      uint32_t bits;
      if (t.dtype == DT_BF16) {
        bits = (uint32_t)h << 16;
      } else {  // IEEE half to single, subnormals, Inf and NaN exactly
        const uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 31, m = h & 1023;
        if (e == 31) {
          bits = sign | 0x7f800000u | (m << 13);
        } else if (e) {
          bits = sign | ((e + 112) << 23) | (m << 13);
        } else if (m) {
          int sh = 0;
          uint32_t mm = m;
          while (!(mm & 1024)) { mm <<= 1; sh++; }
          bits = sign | ((uint32_t)(113 - sh) << 23) | ((mm & 1023) << 13);
        } else {
          bits = sign;
        }
      }
      memcpy(&(*v)[i], &bits, 4);
    }
    ihip_tensor r{v->data(), DT_F32, 0};
    g->widened.push_back(std::move(v));
    return r;
  }
  // a matrix [rows, cols]: the file decides the type (TDecoderModel.Matrix,
  // decoder.pas:2204-2225): blocks in place (scales checked), F32/BF16/F16 in
  // place (the device widens BF16/F16 exactly)
  ihip_tensor matrix(const std::string& name, int64_t rows, int64_t cols)
  {
    const Tensor& t = checked(name, {rows, cols}, true);
    if (block_type(t.dtype)) check_scales(t, name);
    used++;
    return ihip_tensor{t.data, t.dtype, 0};
  }
  // the experts of a layer as one [E, rows, cols] block tensor
  // (TDecoderModel.GgufExperts, decoder.pas:2175-2202)
  // (floats: BF16/F16/F32 in place when `floats`, widened exactly on the device)
  ihip_tensor experts(const std::string& name, int64_t e, int64_t rows, int64_t cols, bool floats = false)
  {
    const Tensor& t = checked(name, {e, rows, cols}, true);
    if (!block_type(t.dtype) && !floats)
      refuse(name + " is " + dtype_name(t.dtype) + ", not supported for experts here");
    if (block_type(t.dtype)) check_scales(t, name);
    used++;
    return ihip_tensor{t.data, t.dtype, 0};
  }

  // TDecoderModel.CheckConfig (decoder.pas:1588-1608), the bounds this path reads
  void check_config(const ihip_model_desc& d) const
  {
    if (d.vocab <= 0 || d.vocab > (1 << 22) || d.hidden <= 0 || d.hidden > (1 << 16) || d.layers <= 0 ||
        d.layers > 1024 || d.heads <= 0 || d.heads > (1 << 12) || d.kv_heads <= 0 || d.kv_heads > d.heads ||
        d.heads % d.kv_heads || d.head_dim <= 0 || d.head_dim > 1024 || (d.head_dim & 1) ||
        (int64_t)d.heads * d.head_dim > (1 << 16) || d.ffn <= 0 || d.ffn > (1 << 18) || d.max_positions <= 0 ||
        d.max_positions > (1 << 24) || !(d.rms_eps > 0) || d.rms_eps > 1 || !(d.rope_theta > 1) ||
        d.rope_theta > 1e12)
      refuse(g->name + " has an invalid or unsupported shape");
    if (d.experts_used && (d.experts_used > d.experts || d.experts > 4096 || d.expert_ffn > (1 << 18)))
      refuse(g->name + " has an invalid or unsupported shape");
  }

  // the settings common to the three architectures
  void common(ihip_model_desc& d, bool qwen, bool qwen2 = false)
  {
    const Tensor* emb = g->tensor("token_embd.weight");
    if (!emb) refuse("no tensor token_embd.weight in " + g->name);
    if (emb->ndim != 2 || emb->shape[0] > (1 << 22))
      refuse(fmt("token_embd.weight is shaped [%lld...] of %d dimensions", (long long)emb->shape[0], emb->ndim));
    d.vocab = (int32_t)emb->shape[0];
    d.hidden = count("embedding_length");
    d.layers = count("block_count");
    d.heads = count("attention.head_count");
    d.kv_heads = count("attention.head_count_kv");
    // qwen2 files name no key length: hidden / heads (HeadDimOf)
    if (!qwen2 || has("attention.key_length")) {
      d.head_dim = count("attention.key_length");
    } else {
      if (d.heads <= 0 || d.hidden <= 0 || d.hidden % d.heads)
        refuse(fmt("a hidden size of %d for %d heads", d.hidden, d.heads));
      d.head_dim = d.hidden / d.heads;
    }
    if (has("rope.dimension_count") && count("rope.dimension_count") != d.head_dim)
      refuse(fmt("RoPE over %d of %d dimensions not supported", count("rope.dimension_count"), d.head_dim));
    if (has("attention.value_length") && count("attention.value_length") != d.head_dim)
      refuse("key and value heads of different sizes");
    d.ffn = count("feed_forward_length");
    d.max_positions = count("context_length");
    d.rms_eps = (float)g->real(arch + ".attention.layer_norm_rms_epsilon");
    d.rope_theta = g->real(arch + ".rope.freq_base");
    (void)qwen;
  }

  // qwen3, qwen3moe and qwen2 (Qwen2 / Qwen2.5: a bias on Q, K and V in
  // place of the head norms, TQwen2Model, model.qwen3.pas:128-139, :635-655)
  void qwen3(ihip_model_desc& d, bool moe, bool qwen2 = false)
  {
    // a scaled RoPE or a sliding window would change the arithmetic: refused
    if (has("rope.scaling.type") && g->str(arch + ".rope.scaling.type") != "none")
      refuse("rope scaling \"" + g->str(arch + ".rope.scaling.type") + "\" not supported");
    if (has("attention.sliding_window")) refuse("sliding window attention not supported");
    common(d, true, qwen2);
    d.swiglu_alpha = 1.0f;
    d.swiglu_limit = 0.0f;
    if (moe) {
      d.experts = count("expert_count");
      d.experts_used = count("expert_used_count");
      d.expert_ffn = count("expert_feed_forward_length");
      d.norm_topk = 1;
    }
    check_config(d);
    const int64_t h = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd, kvw = (int64_t)d.kv_heads * hd;
    d.embed = embedding(d);
    d.final_norm = weight("output_norm.weight", {h});
    // llama.cpp ties the head to the embedding by leaving output.weight out
    d.head = g->tensor("output.weight") ? matrix("output.weight", d.vocab, h) : ihip_tensor{};
    g->layers.assign((size_t)d.layers, ihip_layer_desc{});
    for (int i = 0; i < d.layers; i++) {
      ihip_layer_desc& L = g->layers[i];
      const std::string b = "blk." + std::to_string(i) + ".";
      L.q = matrix(b + "attn_q.weight", qw, h);
      L.k = matrix(b + "attn_k.weight", kvw, h);
      L.v = matrix(b + "attn_v.weight", kvw, h);
      L.o = matrix(b + "attn_output.weight", h, qw);
      if (qwen2) {
        L.q_bias = weight(b + "attn_q.bias", {qw});
        L.k_bias = weight(b + "attn_k.bias", {kvw});
        L.v_bias = weight(b + "attn_v.bias", {kvw});
      } else {
        L.q_norm = weight(b + "attn_q_norm.weight", {hd});
        L.k_norm = weight(b + "attn_k_norm.weight", {hd});
      }
      L.input_norm = weight(b + "attn_norm.weight", {h});
      L.post_norm = weight(b + "ffn_norm.weight", {h});
      // qwen3moe: a layer with a router has experts, the others are dense
      if (moe && g->tensor(b + "ffn_gate_inp.weight")) {
        const int64_t n = d.experts, fi = d.expert_ffn;
        L.moe = 1;
        L.router = matrix(b + "ffn_gate_inp.weight", n, h);
        L.exp_gate = experts(b + "ffn_gate_exps.weight", n, fi, h);
        L.exp_up = experts(b + "ffn_up_exps.weight", n, fi, h);
        L.exp_down = experts(b + "ffn_down_exps.weight", n, h, fi);
      } else {
        L.gate = matrix(b + "ffn_gate.weight", d.ffn, h);
        L.up = matrix(b + "ffn_up.weight", d.ffn, h);
        L.down = matrix(b + "ffn_down.weight", h, d.ffn);
      }
    }
  }

  void gptoss(ihip_model_desc& d)
  {
    common(d, false);
    d.experts = count("expert_count");
    d.experts_used = count("expert_used_count");
    d.expert_ffn = count("expert_feed_forward_length");
    d.norm_topk = 1;
    // llama.cpp: an untied head, the SwiGLU of gpt-oss with fixed settings
    if (!g->tensor("output.weight")) refuse("tied embeddings not supported");
    d.swiglu_limit = 7.0f;
    d.swiglu_alpha = 1.702f;
    // YaRN as the converter writes it: type, factor, original context
    if (g->str(arch + ".rope.scaling.type") != "yarn")
      refuse("rope scaling \"" + g->str(arch + ".rope.scaling.type") + "\" not supported");
    // an attention factor of llama.cpp's own would change the scale: refused
    if (has("rope.scaling.attn_factor") || has("rope.scaling.yarn_log_multiplier"))
      refuse("a YaRN attention factor not supported");
    d.rope_factor = g->real(arch + ".rope.scaling.factor");
    if (!(d.rope_factor > 0)) refuse(fmt("a YaRN factor of %g", d.rope_factor));
    d.rope_original = count("rope.scaling.original_context_length");
    // the betas of the file when it has them, else llama.cpp's defaults
    d.rope_beta_fast = has("rope.scaling.yarn_beta_fast") ? g->real(arch + ".rope.scaling.yarn_beta_fast") : 32.0;
    d.rope_beta_slow = has("rope.scaling.yarn_beta_slow") ? g->real(arch + ".rope.scaling.yarn_beta_slow") : 1.0;
    d.rope_truncate = 0;
    d.rope_attention = 0;
    const int32_t w = count("attention.sliding_window");
    if (w > (1 << 24) || d.layers > 1024)
      refuse(fmt("a sliding window of %d over %d layers", w, d.layers));
    check_config(d);
    const int64_t h = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd, kvw = (int64_t)d.kv_heads * hd;
    const int64_t n = d.experts, fi = d.expert_ffn;
    d.embed = embedding(d);
    d.final_norm = weight("output_norm.weight", {h});
    d.head = matrix("output.weight", d.vocab, h);
    g->layers.assign((size_t)d.layers, ihip_layer_desc{});
    for (int i = 0; i < d.layers; i++) {
      ihip_layer_desc& L = g->layers[i];
      const std::string b = "blk." + std::to_string(i) + ".";
      L.q = matrix(b + "attn_q.weight", qw, h);
      L.k = matrix(b + "attn_k.weight", kvw, h);
      L.v = matrix(b + "attn_v.weight", kvw, h);
      L.o = matrix(b + "attn_output.weight", h, qw);
      L.q_bias = weight(b + "attn_q.bias", {qw});
      L.k_bias = weight(b + "attn_k.bias", {kvw});
      L.v_bias = weight(b + "attn_v.bias", {kvw});
      L.o_bias = weight(b + "attn_output.bias", {h});
      L.sinks = weight(b + "attn_sinks.weight", {d.heads});
      L.input_norm = weight(b + "attn_norm.weight", {h});
      L.post_norm = weight(b + "post_attention_norm.weight", {h});
      L.moe = 1;
      L.router = matrix(b + "ffn_gate_inp.weight", n, h);
      L.router_bias = weight(b + "ffn_gate_inp.bias", {n});
      L.exp_gate = experts(b + "ffn_gate_exps.weight", n, fi, h);
      L.exp_up = experts(b + "ffn_up_exps.weight", n, fi, h);
      L.exp_down = experts(b + "ffn_down_exps.weight", n, h, fi);
      L.exp_gate_bias = weight(b + "ffn_gate_exps.bias", {n, fi});
      L.exp_up_bias = weight(b + "ffn_up_exps.bias", {n, fi});
      L.exp_down_bias = weight(b + "ffn_down_exps.bias", {n, h});
      // llama.cpp: the even layers slide (swa pattern 2)
      if (i % 2 == 0) L.window = w;
    }
  }

  // TQwen35Model.LoadGgufConfig / LoadWeights (model.qwen35.pas:371-452,
  // :534-640): the Gated DeltaNet layers and the gated attention of qwen35
  void qwen35(ihip_model_desc& d)
  {
    // weights folded with a Hadamard transform want it on the activations too
    for (const Value& v : g->values)
      if (v.key.size() >= 6 && strncasecmp(v.key.c_str(), "prism.", 6) == 0)
        refuse(v.key + " (weights of a transformed basis) not supported");
    if (has("rope.scaling.type") && g->str(arch + ".rope.scaling.type") != "none")
      refuse("rope scaling \"" + g->str(arch + ".rope.scaling.type") + "\" not supported");
    if (has("attention.sliding_window")) refuse("sliding window attention not supported");
    const Tensor* emb = g->tensor("token_embd.weight");
    if (!emb) refuse("no tensor token_embd.weight in " + g->name);
    if (emb->ndim != 2 || emb->shape[0] > (1 << 22))
      refuse(fmt("token_embd.weight is shaped [%lld...] of %d dimensions", (long long)emb->shape[0], emb->ndim));
    d.vocab = (int32_t)emb->shape[0];
    d.hidden = count("embedding_length");
    // the multi-token prediction layers follow the model: not computed
    const int32_t blocks = count("block_count");
    const int64_t mtp = has("nextn_predict_layers") ? g->integer(arch + ".nextn_predict_layers") : 0;
    if (mtp < 0 || mtp >= blocks) refuse(fmt("%lld prediction layers of %d blocks", (long long)mtp, blocks));
    d.layers = blocks - (int32_t)mtp;
    d.heads = count("attention.head_count");
    d.kv_heads = count("attention.head_count_kv");
    d.head_dim = count("attention.key_length");
    if (has("attention.value_length") && count("attention.value_length") != d.head_dim)
      refuse("key and value heads of different sizes");
    d.ffn = count("feed_forward_length");
    d.max_positions = count("context_length");
    d.rms_eps = (float)g->real(arch + ".attention.layer_norm_rms_epsilon");
    d.rope_theta = g->real(arch + ".rope.freq_base");
    d.swiglu_alpha = 1.0f;
    d.swiglu_limit = 0.0f;
    d.rope_dims = count("rope.dimension_count");
    if ((d.rope_dims & 1) || d.rope_dims > d.head_dim)
      refuse(fmt("%d rotating values of a head of %d", d.rope_dims, d.head_dim));
    d.lin_conv = count("ssm.conv_kernel");
    d.lin_key_dim = count("ssm.state_size");
    d.lin_key_heads = count("ssm.group_count");
    d.lin_value_heads = count("ssm.time_step_rank");
    const int32_t inner = count("ssm.inner_size");
    if (inner % d.lin_value_heads)
      refuse(fmt("an inner size of %d for %d value heads", inner, d.lin_value_heads));
    d.lin_value_dim = inner / d.lin_value_heads;
    // llama.cpp's converter tiles the value heads when they outnumber the key heads
    d.lin_tiled = d.lin_value_heads != d.lin_key_heads;
    // the kind of every layer: recurrent_layers, else every interval-th is full
    const Value* rl = g->find(arch + ".attention.recurrent_layers");
    if (rl && (rl->vtype != ARR || rl->etype != BOOLV || rl->count != blocks))
      refuse(fmt("attention.recurrent_layers is no array of %d booleans", blocks));
    int32_t interval = 4;
    if (!rl && has("full_attention_interval")) interval = count("full_attention_interval");
    check_config(d);
    bool lin = false;
    std::vector<int> rec((size_t)d.layers);
    for (int i = 0; i < d.layers; i++) {
      rec[i] = rl ? rl->data[i] != 0 : (i + 1) % interval != 0;
      lin = lin || rec[i];
    }
    if (!lin) {
      d.lin_key_heads = d.lin_value_heads = d.lin_key_dim = d.lin_value_dim = d.lin_conv = 0;
      d.lin_tiled = 0;
    } else if (d.lin_key_heads > 1024 || d.lin_value_heads > 1024 || d.lin_value_heads % d.lin_key_heads ||
               d.lin_key_dim > 1024 || d.lin_value_dim > 1024 || d.lin_conv > 64) {
      refuse(fmt("DeltaNet heads of %d x %d (keys) and %d x %d (values) with a convolution of %d",
                 d.lin_key_heads, d.lin_key_dim, d.lin_value_heads, d.lin_value_dim, d.lin_conv));
    }
    const int64_t h = d.hidden, hd = d.head_dim, qw = (int64_t)d.heads * hd, kvw = (int64_t)d.kv_heads * hd;
    const int64_t vh = d.lin_value_heads, vd = vh * d.lin_value_dim,
                  cd = 2 * (int64_t)d.lin_key_heads * d.lin_key_dim + vd, kw = d.lin_conv;
    d.embed = embedding(d);
    d.final_norm = weight("output_norm.weight", {h});
    // llama.cpp ties the head to the embedding by leaving output.weight out
    d.head = g->tensor("output.weight") ? matrix("output.weight", d.vocab, h) : ihip_tensor{};
    g->layers.assign((size_t)d.layers, ihip_layer_desc{});
    for (int i = 0; i < d.layers; i++) {
      ihip_layer_desc& L = g->layers[i];
      const std::string b = "blk." + std::to_string(i) + ".";
      L.input_norm = weight(b + "attn_norm.weight", {h});
      L.post_norm = weight(b + "post_attention_norm.weight", {h});
      L.gate = matrix(b + "ffn_gate.weight", d.ffn, h);
      L.up = matrix(b + "ffn_up.weight", d.ffn, h);
      L.down = matrix(b + "ffn_down.weight", h, d.ffn);
      if (rec[i]) {
        L.mixer = IHIP_MIXER_DELTANET;
        L.lin_qkv = matrix(b + "attn_qkv.weight", cd, h);
        L.lin_z = matrix(b + "attn_gate.weight", vd, h);
        L.lin_b = matrix(b + "ssm_beta.weight", vh, h);
        L.lin_a = matrix(b + "ssm_alpha.weight", vh, h);
        L.lin_out = matrix(b + "ssm_out.weight", h, vd);
        L.lin_conv = weight(b + "ssm_conv1d.weight", {cd, kw});
        L.lin_dt_bias = weight(b + "ssm_dt.bias", {vh});
        // ssm_a holds -exp(A_log): negative and finite, by its bits (a file
        // holding A_log itself would let the state grow instead of decay)
        L.lin_neg_a = weight(b + "ssm_a", {vh});
        for (int64_t j = 0; j < vh; j++) {
          uint32_t bits;
          memcpy(&bits, (const float*)L.lin_neg_a.data + j, 4);
          if (!(bits & 0x80000000u) || (bits & 0x7f800000u) == 0x7f800000u)
            refuse(fmt("blk.%d.ssm_a[%lld] is no -exp(A_log)", i, (long long)j));
        }
        L.lin_norm = weight(b + "ssm_norm.weight", {d.lin_value_dim});
      } else {
        // per head the query rows, then the gate rows
        L.output_gate = 1;
        L.q = matrix(b + "attn_q.weight", 2 * qw, h);
        L.k = matrix(b + "attn_k.weight", kvw, h);
        L.v = matrix(b + "attn_v.weight", kvw, h);
        L.o = matrix(b + "attn_output.weight", h, qw);
        L.q_norm = weight(b + "attn_q_norm.weight", {hd});
        L.k_norm = weight(b + "attn_k_norm.weight", {hd});
      }
    }
    // the tensors of the layers after the model are not the model's
    trunk = 0;
    for (const Tensor& t : g->tensors) {
      int64_t n = -1;
      if (t.name.compare(0, 4, "blk.") == 0) {
        size_t dot = t.name.find('.', 4);
        if (dot != std::string::npos && dot > 4) n = atoll(t.name.substr(4, dot - 4).c_str());
      }
      if (n < d.layers) trunk++;
    }
  }

  // a number of the metadata for layer i: an array of one per layer, or one
  // for all (GgufPerLayer, model.gemma4.pas:477-507)
  int32_t per_layer(const std::string& key, int i, int layers) const
  {
    const Value* v = g->find(arch + "." + key);
    if (!v || v->vtype != ARR) return count(key);
    if (v->count != layers) refuse(fmt("%s has %lld values for %d layers", key.c_str(), (long long)v->count, layers));
    int64_t x;
    if (v->etype == I32) { int32_t t; memcpy(&t, v->data + 4 * i, 4); x = t; }
    else if (v->etype == U32) { uint32_t t; memcpy(&t, v->data + 4 * i, 4); x = t; }
    else refuse(key + " is an array of " + TYPE_NAME[v->etype] + ", expected integers");
    if (x <= 0 || x > (int64_t(1) << 30)) refuse(fmt("%s[%d] = %lld out of range", key.c_str(), i, (long long)x));
    return (int32_t)x;
  }
  // a positive integer of the metadata, or 0 when it is missing
  int64_t int_or0(const std::string& key) const { return has(key) ? g->integer(arch + "." + key) : 0; }

  // TGemma4Model.LoadGgufConfig / LoadWeights (model.gemma4.pas:509-679,
  // :727-860): sliding and full layers of their own heads, two rotary sets,
  // K=V, sandwich norms, GeGLU, the dense block beside the experts
  void gemma4(ihip_model_desc& d)
  {
    // what this family does not compute: per-layer embeddings, shared KV
    // layers, prediction layers, a scaled RoPE, a width per layer, an untied head
    if (int_or0("embedding_length_per_layer_input") != 0) refuse("per-layer embeddings not supported");
    if (int_or0("attention.shared_kv_layers") != 0) refuse("shared KV layers not supported");
    if (int_or0("nextn_predict_layers") != 0) refuse("prediction layers not supported");
    if (has("rope.scaling.type") && g->str(arch + ".rope.scaling.type") != "none")
      refuse("rope scaling \"" + g->str(arch + ".rope.scaling.type") + "\" not supported");
    if (const Value* v = g->find(arch + ".feed_forward_length"))
      if (v->vtype == ARR) refuse("a feed-forward width per layer (the double-wide MLP) not supported");
    if (g->tensor("output.weight")) refuse("an untied head not supported");
    const Tensor* emb = g->tensor("token_embd.weight");
    if (!emb) refuse("no tensor token_embd.weight in " + g->name);
    if (emb->ndim != 2 || emb->shape[0] > (1 << 22))
      refuse(fmt("token_embd.weight is shaped [%lld...] of %d dimensions", (long long)emb->shape[0], emb->ndim));
    d.vocab = (int32_t)emb->shape[0];
    d.hidden = count("embedding_length");
    d.layers = count("block_count");
    if (d.layers > 1024) refuse(fmt("%d layers", d.layers));
    d.heads = count("attention.head_count");
    d.ffn = count("feed_forward_length");
    d.max_positions = count("context_length");
    d.rms_eps = (float)g->real(arch + ".attention.layer_norm_rms_epsilon");
    // the sliding heads (key_length_swa) and the full ones (key_length)
    d.head_dim = count("attention.key_length_swa");
    const int32_t full = count("attention.key_length");
    if (count("attention.value_length_swa") != d.head_dim || count("attention.value_length") != full)
      refuse("key and value heads of different sizes");
    if (count("rope.dimension_count_swa") != d.head_dim || count("rope.dimension_count") != full)
      refuse(fmt("rotating %d and %d values of heads of %d and %d", count("rope.dimension_count_swa"),
                 count("rope.dimension_count"), d.head_dim, full));
    d.rope_theta = g->real(arch + ".rope.freq_base_swa");
    d.rope2_theta = g->real(arch + ".rope.freq_base");
    // rope_freqs: 1 for the rotating pairs of the full head, 1e30 after them
    const Tensor* fr = g->tensor("rope_freqs.weight");
    if (!fr || fr->dtype != DT_F32 || fr->ndim != 1 || fr->shape[0] != full / 2)
      refuse(fmt("rope_freqs.weight is not F32 [%d]", full / 2));
    const float* f = (const float*)fr->data;
    int r = 0;
    while (r < full / 2 && f[r] == 1.0f) r++;
    for (int i = r; i < full / 2; i++)
      if (!(f[i] >= 1e30f))
        refuse(fmt("rope_freqs.weight[%d] = %g is neither 1 before the others nor 1e30 after them", i, f[i]));
    if (r == 0) refuse("rope_freqs.weight rotates no pair");
    used++;
    d.rope2_pairs = r;
    d.activation = IHIP_ACT_GELU_TANH;
    d.attention_scale = 1.0;
    d.value_norm = 1;
    d.swiglu_alpha = 1.0f;
    if (has("final_logit_softcapping")) d.logit_softcap = g->real(arch + ".final_logit_softcapping");
    d.embed_scale = (float)std::sqrt((double)d.hidden);
    if (int_or0("expert_count") != 0) {
      d.experts = count("expert_count");
      d.experts_used = count("expert_used_count");
      d.expert_ffn = count("expert_feed_forward_length");
      d.norm_topk = 1;
    }
    // the kind of every layer: sliding_window_pattern (true: sliding)
    const Value* pat = g->find(arch + ".attention.sliding_window_pattern");
    if (!pat || pat->vtype != ARR || pat->etype != BOOLV || pat->count != d.layers)
      refuse(fmt("attention.sliding_window_pattern is no array of %d booleans", d.layers));
    const int32_t window = count("attention.sliding_window");
    g->layers.assign((size_t)d.layers, ihip_layer_desc{});
    for (int i = 0; i < d.layers; i++) {
      ihip_layer_desc& L = g->layers[i];
      L.kv_heads = per_layer("attention.head_count_kv", i, d.layers);
      if (pat->data[i]) {
        L.window = window;
        if (!d.kv_heads) d.kv_heads = L.kv_heads;
      } else {
        L.head_dim = full;
        L.rope_set = 1;
        // attention_k_eq_v: no attn_v, the values are the keys
        L.k_is_v = g->tensor("blk." + std::to_string(i) + ".attn_v.weight") == nullptr;
      }
      if (L.kv_heads > d.heads || d.heads % L.kv_heads)
        refuse(fmt("layer %d has %d KV heads for %d heads", i, L.kv_heads, d.heads));
    }
    if (!d.kv_heads) refuse("no sliding layer");
    check_config(d);
    if (full > 1024 || full & 1 || (int64_t)d.heads * full > (1 << 16)) refuse(fmt("full heads of %d", full));
    const int64_t h = d.hidden, E = d.experts, fi = d.expert_ffn;
    d.embed = embedding(d);
    d.final_norm = weight("output_norm.weight", {h});
    // the router input: an RMSNorm without weight times scale and hidden^-0.5,
    // folded into one norm weight (float32 products, as the reference)
    const float root = (float)(1 / std::sqrt(1.0 * (double)h));
    for (int i = 0; i < d.layers; i++) {
      ihip_layer_desc& L = g->layers[i];
      const std::string b = "blk." + std::to_string(i) + ".";
      const int64_t hd = L.head_dim ? L.head_dim : d.head_dim, qw = (int64_t)d.heads * hd,
                    kvw = (int64_t)L.kv_heads * hd;
      L.q = matrix(b + "attn_q.weight", qw, h);
      L.k = matrix(b + "attn_k.weight", kvw, h);
      if (!L.k_is_v) L.v = matrix(b + "attn_v.weight", kvw, h);
      L.o = matrix(b + "attn_output.weight", h, qw);
      L.q_norm = weight(b + "attn_q_norm.weight", {hd});
      L.k_norm = weight(b + "attn_k_norm.weight", {hd});
      L.input_norm = weight(b + "attn_norm.weight", {h});
      L.attn_out_norm = weight(b + "post_attention_norm.weight", {h});
      L.post_norm = weight(b + "ffn_norm.weight", {h});
      L.ffn_out_norm = weight(b + "post_ffw_norm.weight", {h});
      L.scalar = weight(b + "layer_output_scale.weight", {1});
      L.gate = matrix(b + "ffn_gate.weight", d.ffn, h);
      L.up = matrix(b + "ffn_up.weight", d.ffn, h);
      L.down = matrix(b + "ffn_down.weight", h, d.ffn);
      if (E > 0) {
        L.moe = IHIP_FFN_DENSE_MOE;
        L.dense_out_norm = weight(b + "post_ffw_norm_1.weight", {h});
        L.moe_in_norm = weight(b + "pre_ffw_norm_2.weight", {h});
        L.moe_out_norm = weight(b + "post_ffw_norm_2.weight", {h});
        L.router = matrix(b + "ffn_gate_inp.weight", E, h);
        const ihip_tensor sc = weight(b + "ffn_gate_inp.scale", {h});
        auto folded = std::make_unique<std::vector<float>>((size_t)h);
        for (int64_t j = 0; j < h; j++) (*folded)[j] = ((const float*)sc.data)[j] * root;
        L.router_norm = ihip_tensor{folded->data(), DT_F32, 0};
        g->widened.push_back(std::move(folded));
        L.expert_scale = weight(b + "ffn_down_exps.scale", {E});
        L.exp_gate = experts(b + "ffn_gate_up_exps.weight", E, 2 * fi, h, true);
        L.exp_gate_up = 1;
        L.exp_down = experts(b + "ffn_down_exps.weight", E, h, fi, true);
      }
    }
  }

  // the token embedding: read per token, so its block scales are checked here
  ihip_tensor embedding(const ihip_model_desc& d)
  {
    const Tensor& t = checked("token_embd.weight", {d.vocab, d.hidden}, true);
    if (block_type(t.dtype)) check_scales(t, "token_embd.weight");
    used++;
    return ihip_tensor{t.data, t.dtype, 0};
  }

  void build()
  {
    ihip_model_desc& d = g->desc;
    d = ihip_model_desc{};
    arch = g->str("general.architecture");
    if (arch == "qwen3") {
      qwen3(d, false);
    } else if (arch == "qwen3moe") {
      qwen3(d, true);
    } else if (arch == "qwen2") {
      qwen3(d, false, true);
    } else if (arch == "gpt-oss") {
      gptoss(d);
    } else if (arch == "qwen35") {
      qwen35(d);
    } else if (arch == "gemma4") {
      gemma4(d);
    } else {
      refuse("architecture \"" + arch + "\" is not supported (qwen3, qwen3moe, qwen2, gpt-oss, qwen35, gemma4)");
    }
    // an unknown tensor means a model this path does not understand
    const int64_t expect = trunk >= 0 ? trunk : (int64_t)g->tensors.size();
    if (used != expect)
      refuse(fmt("%lld tensors of the model in the file, %d understood", (long long)expect, used));
    d.layer = g->layers.data();
    g->have_desc = true;
  }
};

int open_common(ihip_gguf* g, ihip_gguf** out)
{
  try {
    g->parse();
  } catch (const Refused& e) {
    ihip_gguf_close(g);
    return fail(IHIP_E_FORMAT, e.msg);
  } catch (const std::bad_alloc&) {
    ihip_gguf_close(g);
    return fail(IHIP_E_NOMEM, "GGUF: out of host memory");
  }
  *out = g;
  return 0;
}

}  // namespace

extern "C" {

int ihip_gguf_open(const char* path, ihip_gguf** out)
{
  if (!path || !out) return fail(IHIP_E_ARG, "ihip_gguf_open: null argument");
  *out = nullptr;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return fail(IHIP_E_ARG, std::string("GGUF ") + path + ": cannot open: " + strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return fail(IHIP_E_ARG, std::string("GGUF ") + path + ": cannot stat");
  }
  auto* g = new ihip_gguf;
  g->name = path;
  g->size = (int64_t)st.st_size;
  if (g->size > 0) {
    void* p = mmap(nullptr, (size_t)g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      close(fd);
      delete g;
      return fail(IHIP_E_ARG, std::string("GGUF ") + path + ": cannot map");
    }
    g->map = p;
    g->buf = (const uint8_t*)p;
  }
  close(fd);
  return open_common(g, out);
}

int ihip_gguf_open_mem(const void* data, int64_t size, ihip_gguf** out)
{
  if (!out || size < 0 || (size && !data)) return fail(IHIP_E_ARG, "ihip_gguf_open_mem: bad argument");
  *out = nullptr;
  auto* g = new ihip_gguf;
  g->name = "content";
  g->own.assign((const uint8_t*)data, (const uint8_t*)data + size);
  g->buf = g->own.data();
  g->size = size;
  return open_common(g, out);
}

void ihip_gguf_close(ihip_gguf* g)
{
  if (!g) return;
  if (g->map) munmap(g->map, (size_t)g->size);
  delete g;
}

int64_t ihip_gguf_alignment(const ihip_gguf* g) { return g ? g->alignment : -1; }
int64_t ihip_gguf_value_count(const ihip_gguf* g) { return g ? (int64_t)g->values.size() : -1; }
int64_t ihip_gguf_tensor_count(const ihip_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

int ihip_gguf_value_at(const ihip_gguf* g, int64_t i, ihip_gguf_value* out)
{
  if (!g || !out || i < 0 || i >= (int64_t)g->values.size()) return fail(IHIP_E_ARG, "ihip_gguf_value_at");
  const Value& v = g->values[i];
  *out = ihip_gguf_value{v.key.c_str(), v.vtype, v.etype, v.count, v.data};
  return 0;
}

int64_t ihip_gguf_find(const ihip_gguf* g, const char* key)
{
  if (!g || !key) return -1;
  auto it = g->keys.find(key);
  return it == g->keys.end() ? -1 : it->second;
}

// the typed getters raise (return IHIP_E_FORMAT) as TGgufFile's do
#define IHIP_GGUF_TRY(body)                 \
  if (!g || !key) return fail(IHIP_E_ARG, "gguf: null argument"); \
  try {                                     \
    body;                                   \
  } catch (const Refused& e) {              \
    return fail(IHIP_E_FORMAT, e.msg);      \
  }                                         \
  return 0

int ihip_gguf_str(const ihip_gguf* g, const char* key, const char** s, int64_t* len)
{
  IHIP_GGUF_TRY({
    const Value& v = g->value(key, STR);
    memcpy(len, v.data, 8);
    *s = (const char*)v.data + 8;
  });
}

int ihip_gguf_int(const ihip_gguf* g, const char* key, int64_t* v) { IHIP_GGUF_TRY(*v = g->integer(key)); }
int ihip_gguf_float(const ihip_gguf* g, const char* key, double* v) { IHIP_GGUF_TRY(*v = g->real(key)); }
int ihip_gguf_bool(const ihip_gguf* g, const char* key, int* v) { IHIP_GGUF_TRY(*v = g->boolean(key)); }

int ihip_gguf_bool_def(const ihip_gguf* g, const char* key, int def, int* v)
{
  IHIP_GGUF_TRY(*v = g->find(key) ? (int)g->boolean(key) : def);
}

int ihip_gguf_array(const ihip_gguf* g, const char* key, int32_t elem, int64_t count, const void** data,
                    int64_t* n)
{
  IHIP_GGUF_TRY({
    if (elem == STR || elem == ARR) g->refuse(std::string(key) + ": strings are read by ihip_gguf_strings");
    const Value& v = g->array(key, elem, count);
    *data = v.data;
    *n = v.count;
  });
}

int ihip_gguf_strings(const ihip_gguf* g, const char* key, int64_t first, int64_t n, const char** s,
                      int64_t* len)
{
  IHIP_GGUF_TRY({
    const Value& v = g->array(key, STR, -1);
    if (first < 0 || n < 0 || first > v.count || n > v.count - first)
      g->refuse(fmt("%s: strings [%lld, +%lld) of %lld", key, (long long)first, (long long)n, (long long)v.count));
    for (int64_t i = 0; i < n; i++) {
      const uint8_t* p = v.strings[first + i];
      memcpy(&len[i], p, 8);
      s[i] = (const char*)p + 8;
    }
  });
}

int ihip_gguf_tensor_at(const ihip_gguf* g, int64_t i, ihip_gguf_tensor* out)
{
  if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return fail(IHIP_E_ARG, "ihip_gguf_tensor_at");
  const Tensor& t = g->tensors[i];
  out->name = t.name.c_str();
  out->dtype = t.dtype;
  out->ndim = t.ndim;
  for (int j = 0; j < 4; j++) out->shape[j] = t.shape[j];
  out->count = t.count;
  out->bytes = t.bytes;
  out->data = t.data;
  return 0;
}

int64_t ihip_gguf_find_tensor(const ihip_gguf* g, const char* name)
{
  if (!g || !name) return -1;
  auto it = g->names.find(name);
  return it == g->names.end() ? -1 : it->second;
}

int ihip_gguf_weight(const ihip_gguf* g, const char* key, int32_t dtype, int32_t ndim, const int64_t* dims,
                     const void** data)
{
  IHIP_GGUF_TRY({
    const Tensor* t = g->tensor(key);
    if (!t) g->refuse(std::string("no tensor ") + key);
    if (t->dtype != dtype)
      g->refuse(std::string(key) + " is " + dtype_name(t->dtype) + ", expected " + dtype_name(dtype));
    bool ok = t->ndim == ndim && dims;
    for (int j = 0; ok && j < ndim; j++) ok = t->shape[j] == dims[j];
    if (!ok) g->refuse(std::string(key) + " is shaped otherwise");
    *data = t->data;
  });
}

int ihip_gguf_model_desc(ihip_gguf* g, const ihip_model_desc** out)
{
  if (!g || !out) return fail(IHIP_E_ARG, "ihip_gguf_model_desc: null argument");
  *out = nullptr;
  if (!g->have_desc) {
    g->widened.clear();
    g->layers.clear();
    try {
      DescBuilder{g}.build();
    } catch (const Refused& e) {
      return fail(IHIP_E_FORMAT, e.msg);
    }
  }
  *out = &g->desc;
  return 0;
}

}  // extern "C"
