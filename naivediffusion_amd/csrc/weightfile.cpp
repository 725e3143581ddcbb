// Checkpoint files and LoRA folding, on the way into HBM.
//
// Replaces Weights/SafetensorsFile.cs (the memory-mapped reader), the
// narrowing half of Weights/LazyWeights.cs and the merge of
// Weights/LoraFile.cs (LoraMerge.Merge). The file is mapped read-only; a
// tensor goes from the mapping through a pinned, double-buffered staging area
// into device memory with asynchronous copies (the copy of one chunk into
// staging overlaps the DMA of the one before), and any narrowing to the
// model's float width happens on the GPU. A LoRA's low-rank products are
// folded into a weight on the GPU, all of the weight's patches in one pass,
// in the reference's order and rounding.

#include <fcntl.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "runtime.h"

using namespace ndx;

namespace {

// ---- a JSON reader for the safetensors header ------------------------------
//
// The header is one object of objects ({"dtype": str, "shape": [int..],
// "data_offsets": [int, int]}) plus "__metadata__" (string values, though a
// file may carry others, which are skipped). The reader accepts any JSON and
// keeps what the table needs.

struct Json {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  std::string str;
  double num = 0;
  bool integral = false;
  int64_t inum = 0;
  std::vector<Json> items;                              // ARR
  std::vector<std::pair<std::string, Json>> members;    // OBJ
  const Json* get(const char* key) const {
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

struct JsonParser {
  const char* p;
  const char* end;
  int depth = 0;

  [[noreturn]] void bad(const std::string& what) {
    fail(NDX_INVALID_ARG, "the safetensors header is not valid JSON: " + what);
  }
  void ws() {
    while (p < end && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) p++;
  }
  bool lit(const char* s) {
    size_t n = strlen(s);
    if (size_t(end - p) >= n && !memcmp(p, s, n)) {
      p += n;
      return true;
    }
    return false;
  }
  static void utf8(std::string& out, uint32_t c) {
    if (c < 0x80) {
      out += char(c);
    } else if (c < 0x800) {
      out += char(0xC0 | (c >> 6));
      out += char(0x80 | (c & 0x3F));
    } else if (c < 0x10000) {
      out += char(0xE0 | (c >> 12));
      out += char(0x80 | ((c >> 6) & 0x3F));
      out += char(0x80 | (c & 0x3F));
    } else {
      out += char(0xF0 | (c >> 18));
      out += char(0x80 | ((c >> 12) & 0x3F));
      out += char(0x80 | ((c >> 6) & 0x3F));
      out += char(0x80 | (c & 0x3F));
    }
  }
  uint32_t hex4() {
    if (end - p < 4) bad("a short \\u escape");
    uint32_t v = 0;
    for (int i = 0; i < 4; i++) {
      char c = *p++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= c - '0';
      else if (c >= 'a' && c <= 'f') v |= c - 'a' + 10;
      else if (c >= 'A' && c <= 'F') v |= c - 'A' + 10;
      else bad("a bad \\u escape");
    }
    return v;
  }
  std::string string() {
    if (p >= end || *p != '"') bad("a string was expected");
    p++;
    std::string out;
    while (true) {
      if (p >= end) bad("an unterminated string");
      char c = *p++;
      if (c == '"') return out;
      if ((unsigned char)c < 0x20) bad("a control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (p >= end) bad("an unterminated escape");
      char e = *p++;
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
          uint32_t c1 = hex4();
          if (c1 >= 0xD800 && c1 < 0xDC00 && end - p >= 6 && p[0] == '\\' && p[1] == 'u') {
            p += 2;
            uint32_t c2 = hex4();
            if (c2 >= 0xDC00 && c2 < 0xE000) c1 = 0x10000 + ((c1 - 0xD800) << 10) + (c2 - 0xDC00);
          }
          utf8(out, c1);
          break;
        }
        default: bad("an unknown escape");
      }
    }
  }
  Json value() {
    if (++depth > 64) bad("nesting too deep");
    ws();
    if (p >= end) bad("unexpected end");
    Json v;
    char c = *p;
    if (c == '{') {
      v.kind = Json::OBJ;
      p++;
      ws();
      if (p < end && *p == '}') {
        p++;
      } else {
        while (true) {
          ws();
          std::string k = string();
          ws();
          if (p >= end || *p++ != ':') bad("':' was expected");
          v.members.emplace_back(std::move(k), value());
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == '}') {
            p++;
            break;
          }
          bad("',' or '}' was expected");
        }
      }
    } else if (c == '[') {
      v.kind = Json::ARR;
      p++;
      ws();
      if (p < end && *p == ']') {
        p++;
      } else {
        while (true) {
          v.items.push_back(value());
          ws();
          if (p < end && *p == ',') {
            p++;
            continue;
          }
          if (p < end && *p == ']') {
            p++;
            break;
          }
          bad("',' or ']' was expected");
        }
      }
    } else if (c == '"') {
      v.kind = Json::STR;
      v.str = string();
    } else if (lit("true")) {
      v.kind = Json::BOOL;
      v.num = 1;
    } else if (lit("false")) {
      v.kind = Json::BOOL;
    } else if (lit("null")) {
      v.kind = Json::NUL;
    } else if (c == '-' || (c >= '0' && c <= '9')) {
      const char* s = p;
      if (*p == '-') p++;
      while (p < end && *p >= '0' && *p <= '9') p++;
      bool frac = false;
      if (p < end && (*p == '.' || *p == 'e' || *p == 'E')) {
        frac = true;
        p++;
        while (p < end && ((*p >= '0' && *p <= '9') || *p == '+' || *p == '-' || *p == 'e' || *p == 'E')) p++;
      }
      std::string t(s, p);
      if (t == "-" || t.empty()) bad("a bad number");
      v.kind = Json::NUM;
      v.num = strtod(t.c_str(), nullptr);
      if (!frac && t.size() < 19) {
        v.integral = true;
        v.inum = strtoll(t.c_str(), nullptr, 10);
      }
    } else {
      bad(std::string("an unexpected character '") + c + "'");
    }
    depth--;
    return v;
  }
};

// The widths a tensor can be read at (SafetensorsFile.IsSupportedDataType,
// Weights/SafetensorsFile.cs:229-240) as ndx dtypes; -1 for any other.
int parse_dtype(const std::string& d) {
  if (d == "F32") return NDX_F32;
  if (d == "F16") return NDX_F16;
  if (d == "BF16") return NDX_BF16;
  if (d == "U32") return NDX_U32;
  if (d == "I32") return NDX_I32;
  if (d == "U16") return NDX_U16;
  if (d == "I64") return NDX_I64;
  return -1;
}

}  // namespace

struct ndx_safetensors {
  struct Entry {
    std::string name, dtype;
    int64_t shape[8];
    int rank;
    int64_t begin, end;
  };
  int fd = -1;
  const unsigned char* map = nullptr;
  size_t length = 0;
  int64_t data_start = 0;
  std::vector<Entry> entries;
  std::map<std::string, int> index;
  std::vector<std::pair<std::string, std::string>> metadata;
  // Pinned staging for the copies to the device, made on the first read.
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t stage_done[2] = {nullptr, nullptr};
  ndx_device* stage_dev = nullptr;

  void close_all() {
    for (int k = 0; k < 2; k++) {
      if (stage_done[k]) (void)hipEventSynchronize(stage_done[k]);
      if (stage_done[k]) (void)hipEventDestroy(stage_done[k]);
      if (stage[k]) (void)hipHostFree(stage[k]);
      stage_done[k] = nullptr;
      stage[k] = nullptr;
    }
    if (map) munmap((void*)map, length);
    if (fd >= 0) ::close(fd);
    map = nullptr;
    fd = -1;
  }
};

namespace {

constexpr size_t kStageBytes = size_t(32) << 20;

// Parses the header into f's table; every offset is checked against the
// file before anything reads there (SafetensorsFile.ReadHeader :72-149).
void read_header(ndx_safetensors* f) {
  if (f->length < 8) fail(NDX_INVALID_ARG, "the file is too short to be a safetensors file");
  int64_t header_len;
  memcpy(&header_len, f->map, 8);
  if (header_len <= 0 || header_len > int64_t(f->length) - 8 || header_len > INT32_MAX)
    fail(NDX_INVALID_ARG,
         "the safetensors header does not fit the file: it is not a safetensors file, or the download did not "
         "finish");
  f->data_start = 8 + header_len;
  const int64_t data_len = int64_t(f->length) - f->data_start;
  JsonParser jp{(const char*)f->map + 8, (const char*)f->map + 8 + header_len};
  Json root = jp.value();
  jp.ws();
  if (jp.p != jp.end) jp.bad("characters after the table");
  if (root.kind != Json::OBJ) fail(NDX_INVALID_ARG, "the safetensors header is not a tensor table: not an object");
  for (const auto& m : root.members) {
    if (m.first == "__metadata__") {
      if (m.second.kind != Json::OBJ)
        fail(NDX_INVALID_ARG, "the safetensors header is not a tensor table: __metadata__ is not an object");
      // Only the string-valued notes; a later note of the same name wins.
      for (const auto& note : m.second.members) {
        if (note.second.kind != Json::STR) continue;
        bool replaced = false;
        for (auto& kv : f->metadata)
          if (kv.first == note.first) {
            kv.second = note.second.str;
            replaced = true;
          }
        if (!replaced) f->metadata.emplace_back(note.first, note.second.str);
      }
      continue;
    }
    const Json& v = m.second;
    const Json* dt = v.get("dtype");
    const Json* sh = v.get("shape");
    const Json* off = v.get("data_offsets");
    if (v.kind != Json::OBJ || !dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !off ||
        off->kind != Json::ARR || off->items.size() != 2)
      fail(NDX_INVALID_ARG, "the safetensors header is not a tensor table: entry " + m.first);
    ndx_safetensors::Entry e{};
    e.name = m.first;
    e.dtype = dt->str;
    if (sh->items.size() > 8) fail(NDX_INVALID_ARG, "the safetensors entry " + m.first + " has more than 8 axes");
    e.rank = (int)sh->items.size();
    for (int i = 0; i < e.rank; i++) {
      if (!sh->items[i].integral || sh->items[i].inum < 0)
        fail(NDX_INVALID_ARG, "the safetensors header is not a tensor table: a bad extent in " + m.first);
      e.shape[i] = sh->items[i].inum;
    }
    for (const Json& o : off->items)
      if (!o.integral) fail(NDX_INVALID_ARG, "the safetensors header is not a tensor table: a bad offset in " + m.first);
    e.begin = off->items[0].inum;
    e.end = off->items[1].inum;
    if (e.begin < 0 || e.end < e.begin || e.end > data_len)
      fail(NDX_INVALID_ARG, "the safetensors entry " + m.first +
                                " points outside the file: the file is damaged or the download did not finish");
    // A name written twice keeps the later entry, as a JSON object read
    // member by member does.
    auto seen = f->index.find(e.name);
    if (seen != f->index.end()) {
      f->entries[seen->second] = e;
    } else {
      f->index[e.name] = (int)f->entries.size();
      f->entries.push_back(e);
    }
  }
}

const ndx_safetensors::Entry& entry_of(ndx_safetensors* f, const char* name) {
  if (!f->map) fail(NDX_INVALID_STATE, "the file was closed");
  if (!name) fail(NDX_INVALID_ARG, "name is null");
  auto it = f->index.find(name);
  if (it == f->index.end()) fail(NDX_INVALID_ARG, std::string("no tensor ") + name + " in the file");
  return f->entries[it->second];
}

// Copies bytes of the mapping to device memory through the pinned staging
// buffers: chunk k is copied into buffer k % 2 while the DMA of chunk k - 1
// runs; a buffer is reused once its previous DMA has finished.
void upload_mapped(ndx_safetensors* f, ndx_device* dev, const unsigned char* src, size_t bytes, void* dst) {
  if (bytes == 0) return;
  if (f->stage_dev != dev) {
    for (int k = 0; k < 2; k++) {
      if (f->stage_done[k]) {
        (void)hipEventSynchronize(f->stage_done[k]);
        (void)hipEventDestroy(f->stage_done[k]);
        f->stage_done[k] = nullptr;
      }
      if (!f->stage[k]) hip_check(hipHostMalloc(&f->stage[k], kStageBytes, hipHostMallocDefault), "hipHostMalloc");
      hip_check(hipEventCreateWithFlags(&f->stage_done[k], hipEventDisableTiming), "hipEventCreate");
      hip_check(hipEventRecord(f->stage_done[k], dev->stream), "hipEventRecord");
    }
    f->stage_dev = dev;
  }
  size_t done = 0;
  for (int k = 0; done < bytes; k ^= 1) {
    const size_t n = std::min(kStageBytes, bytes - done);
    hip_check(hipEventSynchronize(f->stage_done[k]), "staging");
    memcpy(f->stage[k], src + done, n);
    hip_check(hipMemcpyAsync((char*)dst + done, f->stage[k], n, hipMemcpyHostToDevice, dev->stream), "upload");
    hip_check(hipEventRecord(f->stage_done[k], dev->stream), "hipEventRecord");
    done += n;
  }
  hip_check(hipStreamSynchronize(dev->stream), "upload");
}

View4 flat_view(int64_t n) {
  View4 v;
  for (int i = 0; i < 4; i++) {
    v.size[i] = i == 3 ? n : 1;
    v.stride[i] = i == 3 ? 1 : n;
  }
  return v;
}

int64_t elements_of(const ndx_safetensors::Entry& e) {
  int64_t n = 1;
  for (int i = 0; i < e.rank; i++) n *= e.shape[i];
  return n;
}

}  // namespace

extern "C" {

NDX_API ndx_status ndx_safetensors_open(const char* path, ndx_safetensors** out) {
  NDX_TRY
  if (!path || !out) fail(NDX_INVALID_ARG, "path and out must not be null");
  *out = nullptr;
  auto* f = new ndx_safetensors();
  try {
    f->fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (f->fd < 0) fail(NDX_INVALID_ARG, std::string("cannot open ") + path + ": " + strerror(errno));
    struct stat st;
    if (fstat(f->fd, &st) != 0) fail(NDX_INVALID_ARG, std::string("cannot stat ") + path);
    f->length = size_t(st.st_size);
    if (f->length < 8) fail(NDX_INVALID_ARG, "the file is too short to be a safetensors file");
    void* m = mmap(nullptr, f->length, PROT_READ, MAP_PRIVATE, f->fd, 0);
    if (m == MAP_FAILED) fail(NDX_INVALID_ARG, std::string("cannot map ") + path);
    f->map = (const unsigned char*)m;
    read_header(f);
  } catch (...) {
    // A refused file does not stay mapped (SafetensorsFile.cs:52-62).
    f->close_all();
    delete f;
    throw;
  }
  *out = f;
  NDX_CATCH
}

NDX_API ndx_status ndx_safetensors_close(ndx_safetensors* f) {
  NDX_TRY
  if (!f) return NDX_OK;
  f->close_all();
  delete f;
  NDX_CATCH
}

NDX_API ndx_status ndx_safetensors_count(ndx_safetensors* f, int32_t* entries, int32_t* metadata) {
  NDX_TRY
  NEED(f);
  if (entries) *entries = (int32_t)f->entries.size();
  if (metadata) *metadata = (int32_t)f->metadata.size();
  NDX_CATCH
}

NDX_API ndx_status ndx_safetensors_entry(ndx_safetensors* f, int32_t index, const char** name, const char** dtype,
                                         int64_t* shape, int32_t* rank, uint64_t* bytes) {
  NDX_TRY
  NEED(f);
  if (index < 0 || index >= (int)f->entries.size()) fail(NDX_INVALID_ARG, "no such entry");
  const auto& e = f->entries[index];
  if (name) *name = e.name.c_str();
  if (dtype) *dtype = e.dtype.c_str();
  if (shape)
    for (int i = 0; i < e.rank; i++) shape[i] = e.shape[i];
  if (rank) *rank = e.rank;
  if (bytes) *bytes = uint64_t(e.end - e.begin);
  NDX_CATCH
}

NDX_API ndx_status ndx_safetensors_metadata(ndx_safetensors* f, int32_t index, const char** key, const char** value) {
  NDX_TRY
  NEED(f);
  if (index < 0 || index >= (int)f->metadata.size()) fail(NDX_INVALID_ARG, "no such metadata entry");
  if (key) *key = f->metadata[index].first.c_str();
  if (value) *value = f->metadata[index].second.c_str();
  NDX_CATCH
}

NDX_API ndx_status ndx_safetensors_data(ndx_safetensors* f, const char* name, const void** data, uint64_t* bytes) {
  NDX_TRY
  NEED(f);
  NEED(data);
  const auto& e = entry_of(f, name);
  *data = f->map + f->data_start + e.begin;
  if (bytes) *bytes = uint64_t(e.end - e.begin);
  NDX_CATCH
}

NDX_API ndx_status ndx_safetensors_read(ndx_safetensors* f, const char* name, ndx_device* device, int32_t dtype,
                                        ndx_tensor** out) {
  NDX_TRY
  NEED(f);
  NEED(device);
  NEED(out);
  *out = nullptr;
  device->check_usable();
  const auto& e = entry_of(f, name);
  const int stored = parse_dtype(e.dtype);
  if (stored < 0) fail(NDX_UNSUPPORTED, "safetensors dtype " + e.dtype + " is not supported");
  const int64_t n = elements_of(e);
  if (int64_t(dtype_size(stored)) * n != e.end - e.begin)
    fail(NDX_INVALID_ARG, "the safetensors entry " + e.name + "'s bytes do not match its shape and dtype");
  const int target = dtype < 0 ? stored : dtype;
  if (target != stored && !(dtype_is_float(stored) && dtype_is_float(target)))
    fail(NDX_INVALID_ARG, "only float tensors change width on the way in");
  int64_t shape[4] = {1, 1, 1, 1};
  int rank = e.rank;
  if (rank > 4) {
    // Collapse the leading axes (a [Cout, Cin, kt, kh, kw] video filter).
    int64_t lead = 1;
    for (int i = 0; i + 3 < e.rank; i++) lead *= e.shape[i];
    shape[0] = lead;
    for (int i = 1; i < 4; i++) shape[i] = e.shape[e.rank - 4 + i];
    rank = 4;
  } else {
    for (int i = 0; i < rank; i++) shape[i] = e.shape[i];
  }
  if (rank == 0) {
    rank = 1;
    shape[0] = 1;
  }
  ndx_tensor* raw = new_tensor(device, stored, shape, rank);
  try {
    upload_mapped(f, device, f->map + f->data_start + e.begin, size_t(e.end - e.begin), raw->ptr);
    if (target == stored) {
      *out = raw;
      return NDX_OK;
    }
    ndx_tensor* t = new_tensor(device, target, shape, rank);
    ElemArgs a{};
    a.in0 = raw->ptr;
    a.v0 = flat_view(n);
    a.dt0 = stored;
    a.out = t->ptr;
    a.vo = flat_view(n);
    a.dto = target;
    a.op = ELEM_COPY;
    a.scale = 1.f;
    launch_elementwise(a, device->stream);
    hip_check(hipGetLastError(), "conversion launch");
    hip_check(hipStreamSynchronize(device->stream), "conversion");
    free_tensor(raw);
    *out = t;
  } catch (...) {
    free_tensor(raw);
    throw;
  }
  NDX_CATCH
}

NDX_API ndx_status ndx_lora_fold(const ndx_tensor* weight, const ndx_lora_patch* patches, int32_t count,
                                 int32_t dtype, ndx_tensor** out) {
  NDX_TRY
  NEED(weight);
  NEED(out);
  *out = nullptr;
  if (count < 0 || count > kMaxLoraPatches)
    fail(NDX_INVALID_ARG, "a fold takes 0 to " + std::to_string(kMaxLoraPatches) + " pairs");
  if (count > 0) NEED(patches);
  ndx_device* dev = weight->dev;
  dev->check_usable();
  if (!dtype_is_float(weight->dtype)) fail(NDX_INVALID_ARG, "the weight must be a float tensor");
  // The reference's width: float32 stays float32, anything else comes out
  // as float16 (LoraFile.cs:380-382).
  const int target = dtype < 0 ? (weight->dtype == NDX_F32 ? NDX_F32 : NDX_F16) : dtype;
  if (!dtype_is_float(target)) fail(NDX_INVALID_ARG, "the folded weight is Float32, Float16 or BFloat16");
  const int64_t rows = weight->rank ? weight->shape[0] : 1;
  if (rows == 0) fail(NDX_INVALID_ARG, "the weight has no rows");
  const int64_t cols = weight->numel() / rows;
  LoraFoldArgs a{};
  a.w = weight->ptr;
  a.w_dtype = weight->dtype;
  a.rows = rows;
  a.cols = cols;
  a.out_dtype = target;
  a.patches = count;
  for (int k = 0; k < count; k++) {
    const ndx_lora_patch& p = patches[k];
    NEED(p.down);
    NEED(p.up);
    if (p.down->dev != dev || p.up->dev != dev) fail(NDX_INVALID_ARG, "a pair lives on another device");
    if (!dtype_is_float(p.down->dtype) || !dtype_is_float(p.up->dtype))
      fail(NDX_INVALID_ARG, "a pair's matrices must be float tensors");
    // LoraMerge.Check (LoraFile.cs:342-355): down is [rank, the weight's
    // row], up is [rows covered, rank].
    const int64_t rank = p.down->rank ? p.down->shape[0] : 0;
    const int64_t covered = p.up->rank ? p.up->shape[0] : 0;
    if (rank <= 0 || rank > INT32_MAX || p.down->numel() != rank * cols || p.up->numel() != covered * rank)
      fail(NDX_INVALID_ARG, "pair " + std::to_string(k) + " is not the shape of the weight's rows");
    if (p.first_row < 0 || p.first_row + covered > rows)
      fail(NDX_INVALID_ARG, "pair " + std::to_string(k) + " covers rows the weight does not have");
    a.p[k].down = p.down->ptr;
    a.p[k].up = p.up->ptr;
    a.p[k].down_dtype = p.down->dtype;
    a.p[k].up_dtype = p.up->dtype;
    a.p[k].rank = (int)rank;
    a.p[k].first = p.first_row;
    a.p[k].count = covered;
    a.p[k].scale = p.scale;
  }
  ndx_tensor* t = new_tensor(dev, target, weight->shape, weight->rank);
  try {
    a.out = t->ptr;
    launch_lora_fold(a, dev->stream);
    hip_check(hipGetLastError(), "lora fold launch");
    hip_check(hipStreamSynchronize(dev->stream), "lora fold");
  } catch (...) {
    free_tensor(t);
    throw;
  }
  *out = t;
  NDX_CATCH
}

}  // extern "C"
