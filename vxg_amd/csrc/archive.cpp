// archive.cpp -- host-side readers for the two weight containers the path
// loads from, and device upload straight from their bytes.
//
// .vxt (VXT1), format.rs:296-451 (reader), :178-294 (writer), format_io.rs:
//   "VXT1" | u32 version (1) | u32 tensor count | u32 metadata count
//   metadata: count x { u32 key_len, key, u64 len, value }   (value raw or VXLZ)
//   tensors:  count x { pad to 64 | u32 name_len, name | u8 kind, u8 sub,
//                       6 pad | u64 rows, cols, padded_cols | planes |
//                       u64 FNV-1a64 of the section }
//   u64 FNV-1a64 of everything before it.
// Planes are u64 element counts followed by little-endian data.  The reader
// checks both tags and, for KIND_CODEBOOK, the header and plane rules of
// format.rs:421-451 and the CSR rules of format.rs:565-574.  Sections of the
// other kinds with a fixed plane sequence are stepped over (their planes are
// not validated: nothing here consumes them); a KIND_TURBO_WHT_EC section,
// whose length is only known to its entropy decoder, stops the walk with
// VXT_E_UNSUPPORTED.
//
// GGUF v2/v3, gguf.rs:75-172: "GGUF" | u32 version | u64 tensor count | u64
// kv count | kv table (general.alignment read, the rest skipped by type) |
// tensor infos { string name, u32 n_dims, u64 ne[n_dims], u32 type, u64
// offset } | data section at the next multiple of the alignment.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/vxt_hip.h"

namespace {

struct Fail {
  int code;
  std::string msg;
};

[[noreturn]] void fail(int code, const std::string& msg) { throw Fail{code, msg}; }

void set_err(char* err, size_t cap, const std::string& msg) {
  if (!err || cap == 0) return;
  std::snprintf(err, cap, "%s", msg.c_str());
}

template <typename F>
int guarded(char* err, size_t cap, F&& f) {
  if (err && cap) err[0] = '\0';
  try {
    f();
    return VXT_OK;
  } catch (const Fail& e) {
    set_err(err, cap, e.msg);
    return e.code;
  } catch (const std::bad_alloc&) {
    set_err(err, cap, "out of host memory");
    return VXT_E_DEVICE;
  } catch (...) {
    set_err(err, cap, "unexpected error");
    return VXT_E_DEVICE;
  }
}

uint64_t fnv1a64(const uint8_t* p, size_t n) {
  uint64_t h = 0xcbf29ce484222325ull;
  for (size_t i = 0; i < n; ++i) {
    h ^= p[i];
    h *= 0x100000001b3ull;
  }
  return h;
}

// Bounds-checked little-endian cursor over [0, len).
struct Cursor {
  const uint8_t* b;
  size_t len, pos;
  const char* what;

  void need(size_t n) const {
    if (n > len - pos) fail(VXT_E_FORMAT, std::string("truncated ") + what);
  }
  const uint8_t* take(size_t n) {
    need(n);
    const uint8_t* p = b + pos;
    pos += n;
    return p;
  }
  uint8_t u8() { return *take(1); }
  uint32_t u32() {
    uint32_t v;
    std::memcpy(&v, take(4), 4);
    return v;
  }
  uint64_t u64() {
    uint64_t v;
    std::memcpy(&v, take(8), 8);
    return v;
  }
  void align64() {
    const size_t rem = pos % 64;
    if (rem) take(64 - rem);
  }
  // A plane: u64 count, then count * esz bytes.  Returns the data offset.
  uint64_t plane(size_t esz, uint64_t* count) {
    const uint64_t n = u64();
    if (n > (len - pos) / esz) fail(VXT_E_FORMAT, std::string("truncated ") + what);
    const uint64_t off = pos;
    pos += n * esz;
    *count = n;
    return off;
  }
};

constexpr uint8_t kKindLossless = 1, kKindCodebook = 2, kKindQ40 = 3, kKindWht2 = 4, kKindRawF32 = 5,
                  kKindTurboWht = 6, kKindTurboWhtEc = 7;

uint32_t rd32(const uint8_t* p) {
  uint32_t v;
  std::memcpy(&v, p, 4);
  return v;
}

void parse_vxt(const uint8_t* bytes, size_t len, std::vector<VxtArchiveEntry>* out, uint32_t* meta_count) {
  if (!bytes) fail(VXT_E_ARG, "null archive");
  if (len < 24) fail(VXT_E_FORMAT, "truncated VXT archive");
  if (std::memcmp(bytes, "VXT1", 4) != 0) fail(VXT_E_FORMAT, "invalid VXT magic (expected VXT1)");
  if (rd32(bytes + 4) != 1) fail(VXT_E_UNSUPPORTED, "unsupported VXT version " + std::to_string(rd32(bytes + 4)));
  const size_t body = len - 8;
  uint64_t tag;
  std::memcpy(&tag, bytes + body, 8);
  if (fnv1a64(bytes, body) != tag) fail(VXT_E_FORMAT, "VXT archive checksum mismatch");
  Cursor r{bytes, body, 8, "VXT archive"};
  const uint32_t count = r.u32();
  const uint32_t mcount = r.u32();
  for (uint32_t i = 0; i < mcount; ++i) {
    r.take(r.u32());
    uint64_t n;
    r.plane(1, &n);
  }
  if (meta_count) *meta_count = mcount;
  for (uint32_t i = 0; i < count; ++i) {
    r.align64();
    VxtArchiveEntry e{};
    const size_t section_start = r.pos;
    e.name_len = r.u32();
    e.name_off = r.pos;
    r.take(e.name_len);
    e.kind = r.u8();
    e.sub = r.u8();
    r.take(6);
    e.rows = r.u64();
    e.cols = r.u64();
    e.padded_cols = r.u64();
    if (e.rows == 0 || e.cols == 0 || e.padded_cols < e.cols) fail(VXT_E_FORMAT, "invalid VXT matrix dimensions");
    // format.rs:355-366: every plane-size product must stay far from overflow.
    if (e.cols > (1ull << 40) || e.padded_cols > (1ull << 40) || e.rows > (1ull << 40) ||
        ((e.rows + 3) / 4 * 4) > (uint64_t)(INT64_MAX / 4) / e.padded_cols)
      fail(VXT_E_FORMAT, "VXT matrix dimensions overflow");
    uint64_t n;
    switch (e.kind) {
      case kKindCodebook: {
        if ((e.sub != 3 && e.sub != 4) || e.padded_cols != (e.cols + 255) / 256 * 256)
          fail(VXT_E_FORMAT, "invalid VXT codebook header");
        e.centroids_off = r.pos;
        r.take(64);
        e.scales_off = r.plane(2, &e.n_scales);
        e.words_off = r.plane(4, &e.n_words);
        e.row_ptr_off = r.plane(4, &e.n_row_ptr);
        e.outliers_off = r.plane(4, &e.n_outliers);
        const uint64_t groups = e.rows * (e.padded_cols / 128);
        if (e.n_scales != groups || e.n_words != groups * 4u * e.sub || e.n_row_ptr != e.rows + 1 ||
            rd32(bytes + e.row_ptr_off + 4 * e.rows) != e.n_outliers)
          fail(VXT_E_FORMAT, "corrupt VXT codebook plane lengths");
        // format.rs:565-574
        const uint8_t* rp = bytes + e.row_ptr_off;
        bool ok = rd32(rp) == 0;
        for (uint64_t k = 0; ok && k < e.rows; ++k) {
          const uint32_t a = rd32(rp + 4 * k), b = rd32(rp + 4 * k + 4);
          ok = a <= b && b <= e.n_outliers;
        }
        for (uint64_t k = 0; ok && k < e.n_outliers; ++k) ok = (rd32(bytes + e.outliers_off + 4 * k) & 0xffffu) < e.cols;
        if (!ok) fail(VXT_E_FORMAT, "invalid VXT outlier CSR indices");
        break;
      }
      case kKindLossless:
        r.take(8);
        r.plane(1, &n);
        r.plane(4, &n);
        r.plane(4, &n);
        r.plane(1, &n);
        break;
      case kKindQ40: {
        // format.rs:453-462
        if (e.padded_cols != (e.cols + 31) / 32 * 32) fail(VXT_E_FORMAT, "invalid VXT Q4_0 padded_cols");
        e.scales_off = r.plane(2, &e.n_scales);
        e.words_off = r.plane(4, &e.n_words);
        const uint64_t blocks = e.rows * (e.padded_cols / 32);
        if (e.n_scales != blocks || e.n_words != blocks * 4u) fail(VXT_E_FORMAT, "corrupt VXT Q4_0 plane lengths");
        break;
      }
      case kKindWht2:
        r.take(64);
        r.plane(2, &n);
        r.plane(4, &n);
        r.plane(4, &n);
        r.plane(4, &n);
        break;
      case kKindRawF32:
        r.plane(4, &n);
        break;
      case kKindTurboWht:
        r.plane(2, &n);
        r.plane(4, &n);
        break;
      case kKindTurboWhtEc:
        fail(VXT_E_UNSUPPORTED, "entropy-coded TurboWht sections cannot be stepped over by this reader");
      default:
        fail(VXT_E_FORMAT, "unknown VXT tensor kind " + std::to_string(e.kind));
    }
    e.section_off = section_start;
    e.section_len = r.pos - section_start;
    const uint64_t sect_tag = r.u64();
    if (fnv1a64(bytes + section_start, e.section_len) != sect_tag)
      fail(VXT_E_FORMAT, "VXT integrity mismatch on tensor '" +
                             std::string(reinterpret_cast<const char*>(bytes + e.name_off), e.name_len) + "'");
    out->push_back(e);
  }
}

std::string gguf_str(Cursor& r) {
  const uint64_t n = r.u64();
  if (n > r.len - r.pos) fail(VXT_E_FORMAT, "truncated GGUF string");
  return std::string(reinterpret_cast<const char*>(r.take(n)), n);
}

void skip_gguf_val(Cursor& r, uint32_t vtype, int depth) {
  if (depth > 4) fail(VXT_E_FORMAT, "GGUF arrays nested too deep");
  switch (vtype) {
    case 0: case 1: case 7: r.take(1); break;
    case 2: case 3: r.take(2); break;
    case 4: case 5: case 6: r.take(4); break;
    case 8: {
      const uint64_t n = r.u64();
      if (n > r.len - r.pos) fail(VXT_E_FORMAT, "truncated GGUF string");
      r.take(n);
      break;
    }
    case 9: {
      const uint32_t et = r.u32();
      const uint64_t n = r.u64();
      if (n > r.len - r.pos) fail(VXT_E_FORMAT, "GGUF array longer than the file");
      for (uint64_t k = 0; k < n; ++k) skip_gguf_val(r, et, depth + 1);
      break;
    }
    case 10: case 11: case 12: r.take(8); break;
    default: fail(VXT_E_FORMAT, "unknown GGUF metadata value type " + std::to_string(vtype));
  }
}

// gguf.rs:32-41
bool ggml_bytes(uint32_t type, uint64_t numel, uint64_t* bytes) {
  switch (type) {
    case 0: *bytes = numel * 4; return numel <= UINT64_MAX / 4;
    case 1: case 30: *bytes = numel * 2; return numel <= UINT64_MAX / 2;
    case 2: *bytes = numel / 32 * 18; return numel % 32 == 0;
    case 8: *bytes = numel / 32 * 34; return numel % 32 == 0;
    case 12: *bytes = numel / 256 * 144; return numel % 256 == 0;
    default: return false;
  }
}

void parse_gguf(const uint8_t* bytes, size_t len, std::vector<VxtGgufTensor>* out, uint32_t* version,
                uint64_t* alignment) {
  if (!bytes) fail(VXT_E_ARG, "null GGUF file");
  Cursor r{bytes, len, 0, "GGUF file"};
  if (len < 4 || std::memcmp(r.take(4), "GGUF", 4) != 0) fail(VXT_E_FORMAT, "not a GGUF file (missing GGUF magic)");
  const uint32_t ver = r.u32();
  if (ver < 2 || ver > 3) fail(VXT_E_UNSUPPORTED, "unsupported GGUF version " + std::to_string(ver));
  const uint64_t tcount = r.u64();
  const uint64_t kvcount = r.u64();
  uint64_t align = 32;
  for (uint64_t k = 0; k < kvcount; ++k) {
    const std::string key = gguf_str(r);
    const uint32_t vt = r.u32();
    if (key == "general.alignment" && (vt == 4 || vt == 10)) {
      const uint64_t a = vt == 4 ? r.u32() : r.u64();
      if (a > 0 && (a & (a - 1)) == 0) align = a;
    } else {
      skip_gguf_val(r, vt, 0);
    }
  }
  if (tcount > (len - r.pos) / 24) fail(VXT_E_FORMAT, "GGUF tensor count larger than the file");
  std::vector<VxtGgufTensor> ts;
  for (uint64_t k = 0; k < tcount; ++k) {
    VxtGgufTensor t{};
    const uint64_t nlen = r.u64();
    if (nlen > r.len - r.pos) fail(VXT_E_FORMAT, "truncated GGUF string");
    t.name_off = r.pos;
    t.name_len = nlen;
    r.take(nlen);
    t.n_dims = r.u32();
    if (t.n_dims > 8) fail(VXT_E_FORMAT, "GGUF tensor n_dims > 8");
    for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = r.u64();
    t.ggml_type = r.u32();
    t.data_off = r.u64();   // relative for now
    ts.push_back(t);
  }
  const uint64_t data_start = (r.pos + align - 1) / align * align;
  if (data_start > len) fail(VXT_E_FORMAT, "GGUF data_start past EOF");
  for (auto& t : ts) {
    uint64_t numel = 1;
    for (uint32_t d = 0; d < t.n_dims; ++d) {
      if (t.ne[d] != 0 && numel > UINT64_MAX / t.ne[d]) fail(VXT_E_FORMAT, "GGUF dimension overflow");
      numel *= t.ne[d];
    }
    uint64_t nbytes = 0;
    t.supported = ggml_bytes(t.ggml_type, numel, &nbytes) ? 1u : 0u;
    t.data_len = t.supported ? nbytes : 0;
    if (t.supported) {   // gguf.rs:160-172
      if (t.data_off > len - data_start || t.data_len > len - data_start - t.data_off)
        fail(VXT_E_FORMAT, "GGUF tensor slice past EOF");
    }
    t.data_off += data_start;
  }
  *out = std::move(ts);
  if (version) *version = ver;
  if (alignment) *alignment = align;
}

template <typename T>
std::vector<T> copy_plane(const uint8_t* bytes, uint64_t off, uint64_t n) {
  std::vector<T> v(n);
  if (n) std::memcpy(v.data(), bytes + off, n * sizeof(T));
  return v;
}

}  // namespace

extern "C" {

int vxt_hip_vxt_parse(const uint8_t* bytes, size_t len, VxtArchiveEntry* entries, uint32_t cap, uint32_t* count,
                      uint32_t* meta_count, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    std::vector<VxtArchiveEntry> es;
    parse_vxt(bytes, len, &es, meta_count);
    if (count) *count = (uint32_t)es.size();
    if (entries) {
      if (cap < es.size()) fail(VXT_E_ARG, "entry array too small");
      std::memcpy(entries, es.data(), es.size() * sizeof(VxtArchiveEntry));
    }
  });
}

void* vxt_hip_upload_vxt_entry(void* ctx, const uint8_t* bytes, size_t len, const VxtArchiveEntry* e, char* err,
                               size_t err_cap) {
  void* out = nullptr;
  int rc = guarded(err, err_cap, [&] {
    if (!bytes || !e) fail(VXT_E_ARG, "null archive or entry");
    if (e->kind != kKindCodebook && e->kind != kKindQ40)
      fail(VXT_E_UNSUPPORTED, "only codebook (KIND_CODEBOOK) and Q4_0 entries upload");
    if (e->rows > 0xffffffffu || e->cols > 0xffffffffu || e->padded_cols > 0xffffffffu)
      fail(VXT_E_SHAPE, "matrix too large");
    if (e->kind == kKindQ40) {
      if (e->scales_off + 2 * e->n_scales > len || e->words_off + 4 * e->n_words > len)
        fail(VXT_E_ARG, "entry does not describe this archive");
      const auto sc = copy_plane<uint16_t>(bytes, e->scales_off, e->n_scales);
      const auto wd = copy_plane<uint32_t>(bytes, e->words_off, e->n_words);
      char e2[512];
      out = vxt_hip_upload_q4_0(ctx, (uint32_t)e->rows, (uint32_t)e->cols, (uint32_t)e->padded_cols, sc.data(),
                                sc.size(), wd.data(), wd.size(), e2, sizeof(e2));
      if (!out) fail(VXT_E_FORMAT, e2);
      return;
    }
    if (e->sub != 4) fail(VXT_E_UNSUPPORTED, "only 4-bit codebooks run on the device");
    const uint64_t ends[] = {e->centroids_off + 64, e->scales_off + 2 * e->n_scales, e->words_off + 4 * e->n_words,
                             e->row_ptr_off + 4 * e->n_row_ptr, e->outliers_off + 4 * e->n_outliers};
    for (uint64_t x : ends)
      if (x > len) fail(VXT_E_ARG, "entry does not describe this archive");
    // Planes sit at arbitrary byte offsets in the archive: aligned copies.
    const auto cent = copy_plane<float>(bytes, e->centroids_off, 16);
    const auto sc = copy_plane<uint16_t>(bytes, e->scales_off, e->n_scales);
    const auto wd = copy_plane<uint32_t>(bytes, e->words_off, e->n_words);
    const auto rp = copy_plane<uint32_t>(bytes, e->row_ptr_off, e->n_row_ptr);
    const auto ol = copy_plane<uint32_t>(bytes, e->outliers_off, e->n_outliers);
    VxtCb4View v{4u, (uint32_t)e->rows, (uint32_t)e->cols, (uint32_t)e->padded_cols, cent.data(), sc.data(),
                 sc.size(), wd.data(), wd.size(), rp.data(), rp.size(), ol.empty() ? nullptr : ol.data(), ol.size()};
    char e2[512];
    out = vxt_hip_upload_cb4(ctx, &v, e2, sizeof(e2));
    if (!out) fail(VXT_E_FORMAT, e2);
  });
  return rc == VXT_OK ? out : nullptr;
}

int vxt_hip_gguf_parse(const uint8_t* bytes, size_t len, VxtGgufTensor* tensors, uint32_t cap, uint32_t* count,
                       uint32_t* version, uint64_t* alignment, char* err, size_t err_cap) {
  return guarded(err, err_cap, [&] {
    std::vector<VxtGgufTensor> ts;
    parse_gguf(bytes, len, &ts, version, alignment);
    if (ts.size() > 0xffffffffu) fail(VXT_E_FORMAT, "too many GGUF tensors");
    if (count) *count = (uint32_t)ts.size();
    if (tensors) {
      if (cap < ts.size()) fail(VXT_E_ARG, "tensor array too small");
      std::memcpy(tensors, ts.data(), ts.size() * sizeof(VxtGgufTensor));
    }
  });
}

void* vxt_hip_upload_gguf_q8_0(void* ctx, const uint8_t* bytes, size_t len, const VxtGgufTensor* t, char* err,
                               size_t err_cap) {
  void* out = nullptr;
  int rc = guarded(err, err_cap, [&] {
    if (!bytes || !t) fail(VXT_E_ARG, "null file or tensor");
    if (t->ggml_type != 8) fail(VXT_E_UNSUPPORTED, "only Q8_0 GGUF tensors upload directly");
    if (t->n_dims < 2 || t->n_dims > 8) fail(VXT_E_SHAPE, "a matrix needs at least two dimensions");
    // gguf.rs:65-73: ne[0] is the contiguous cols, the rest multiply to rows.
    uint64_t rows = 1;
    for (uint32_t d = 1; d < t->n_dims; ++d) rows *= t->ne[d];
    const uint64_t cols = t->ne[0];
    if (rows == 0 || cols == 0 || cols % 32 != 0) fail(VXT_E_SHAPE, "Q8_0 rows need cols % 32 == 0");
    if (rows > 0xffffffffu || cols > 0xffffffffu) fail(VXT_E_SHAPE, "matrix too large");
    if (t->data_off > len || t->data_len > len - t->data_off || t->data_len != rows * cols / 32 * 34)
      fail(VXT_E_ARG, "tensor does not describe this file");
    char e2[512];
    out = vxt_hip_upload_q8_0(ctx, (uint32_t)rows, (uint32_t)cols, bytes + t->data_off, t->data_len, e2, sizeof(e2));
    if (!out) fail(VXT_E_FORMAT, e2);
  });
  return rc == VXT_OK ? out : nullptr;
}

}  // extern "C"
