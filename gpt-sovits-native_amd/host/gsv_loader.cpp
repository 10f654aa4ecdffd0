// gsv_loader.cpp — the .gsv (GSV1) weight container: read-only mapping, header and directory
// validation with the reference loader's rules, and the upload of each segment kind to the GPU as
// one contiguous device arena (one host-to-device copy instead of one per tensor).
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "gsvk.h"
#include "gsvk_gsv.h"

namespace {

constexpr uint64_t kAlign = 64;
constexpr uint64_t kMaxNumel = 1ull << 40;
constexpr uint32_t kVersion = 1;
constexpr uint32_t kFlagHasF16 = 1u;

struct Reader {
  const uint8_t* p;
  const uint8_t* end;
  bool ok = true;
  const uint8_t* take(size_t n) {
    if (!ok || static_cast<size_t>(end - p) < n) {
      ok = false;
      return nullptr;
    }
    const uint8_t* r = p;
    p += n;
    return r;
  }
  template <class T>
  T get() {
    T v{};
    if (const uint8_t* q = take(sizeof(T))) std::memcpy(&v, q, sizeof(T));
    return v;
  }
};

}  // namespace

struct gsvk_gsv {
  const uint8_t* base = nullptr;
  uint64_t size = 0;
  void* map = nullptr;  // owned mapping (gsvk_gsv_open) or nullptr (caller's buffer)
  uint32_t version = 0, flags = 0, n_tensors = 0;
  const char* name = nullptr;
  size_t name_len = 0;
  const char* config = nullptr;
  size_t config_len = 0;
  std::vector<gsvk_gsv_tensor> t;
};

namespace {

// Header (parse_gsv_raw_header, gsv_header.cpp:29-56) and directory (parse_gsv_directory,
// gsv_loader.cpp:46-108); every rule the reference checks makes the file GSVK_E_FORMAT.
int parse(gsvk_gsv* g) {
  Reader r{g->base, g->base + g->size};
  const uint8_t* magic = r.take(4);
  if (!magic || std::memcmp(magic, "GSV1", 4) != 0) return GSVK_E_FORMAT;
  g->version = r.get<uint32_t>();
  g->flags = r.get<uint32_t>();
  if (!r.ok || g->version != kVersion) return GSVK_E_FORMAT;
  const uint16_t nl = r.get<uint16_t>();
  g->name = reinterpret_cast<const char*>(r.take(nl));
  g->name_len = nl;
  const uint32_t cl = r.get<uint32_t>();
  g->config = reinterpret_cast<const char*>(r.take(cl));
  g->config_len = cl;
  g->n_tensors = r.get<uint32_t>();
  if (!r.ok) return GSVK_E_FORMAT;
  bool any_f16 = false;
  for (uint32_t i = 0; i < g->n_tensors; ++i) {
    gsvk_gsv_tensor t{};
    const uint16_t tl = r.get<uint16_t>();
    t.name = reinterpret_cast<const char*>(r.take(tl));
    t.name_len = tl;
    t.rank = r.get<uint16_t>();
    if (!r.ok || t.rank > 8) return GSVK_E_FORMAT;
    uint64_t numel = 1;
    for (uint32_t d = 0; d < t.rank; ++d) {
      t.dims[d] = r.get<uint32_t>();
      // checked before the multiply: numel <= 2^40 times a dim below 2^32 could wrap 64 bits
      if (t.dims[d] != 0 && numel > kMaxNumel / t.dims[d]) return GSVK_E_FORMAT;
      numel *= t.dims[d];
    }
    t.numel = numel;
    t.src_dtype = r.get<uint16_t>();
    t.f32_offset = r.get<uint64_t>();
    t.f32_nbytes = r.get<uint64_t>();
    t.f16_offset = r.get<uint64_t>();
    t.f16_nbytes = r.get<uint64_t>();
    if (!r.ok || (t.src_dtype != 1 && t.src_dtype != 2)) return GSVK_E_FORMAT;
    const bool has16 = t.f16_nbytes != 0;
    // an fp32 segment of the shape's size, or none at all next to an fp16 copy (slim files)
    if (has16 ? (t.f32_nbytes != 0 && t.f32_nbytes != numel * 4) : t.f32_nbytes != numel * 4)
      return GSVK_E_FORMAT;
    if (has16 && t.f16_nbytes != numel * 2) return GSVK_E_FORMAT;
    if (t.f32_nbytes != 0 &&
        (t.f32_offset % kAlign || t.f32_offset > g->size || t.f32_nbytes > g->size - t.f32_offset))
      return GSVK_E_FORMAT;
    if (has16 &&
        (t.f16_offset % kAlign || t.f16_offset > g->size || t.f16_nbytes > g->size - t.f16_offset))
      return GSVK_E_FORMAT;
    any_f16 = any_f16 || has16;
    g->t.push_back(t);
  }
  if (((g->flags & kFlagHasF16) != 0) != any_f16) return GSVK_E_FORMAT;
  return GSVK_OK;
}

int finish_open(gsvk_gsv* g, gsvk_gsv** out) {
  const int rc = parse(g);
  if (rc != GSVK_OK) {
    gsvk_gsv_close(g);
    return rc;
  }
  *out = g;
  return GSVK_OK;
}

bool seg(const gsvk_gsv_tensor& t, int kind, uint64_t& off, uint64_t& nb) {
  if (kind == GSVK_F16) {
    off = t.f16_offset;
    nb = t.f16_nbytes;
  } else {
    off = t.f32_offset;
    nb = t.f32_nbytes;
  }
  return nb != 0;
}

}  // namespace

extern "C" int gsvk_gsv_open(const char* path, gsvk_gsv** out) {
  if (!path || !out) return GSVK_E_NULL;
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return GSVK_E_IO;
  struct stat st {};
  if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
    ::close(fd);
    return GSVK_E_IO;
  }
  void* m = ::mmap(nullptr, static_cast<size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);  // the mapping stays valid
  if (m == MAP_FAILED) return GSVK_E_IO;
  auto* g = new (std::nothrow) gsvk_gsv;
  if (!g) {
    ::munmap(m, static_cast<size_t>(st.st_size));
    return GSVK_E_IO;
  }
  g->map = m;
  g->base = static_cast<const uint8_t*>(m);
  g->size = static_cast<uint64_t>(st.st_size);
  return finish_open(g, out);
}

extern "C" int gsvk_gsv_open_memory(const void* data, size_t size, gsvk_gsv** out) {
  if (!data || !out) return GSVK_E_NULL;
  *out = nullptr;
  auto* g = new (std::nothrow) gsvk_gsv;
  if (!g) return GSVK_E_IO;
  g->base = static_cast<const uint8_t*>(data);
  g->size = size;
  return finish_open(g, out);
}

extern "C" void gsvk_gsv_close(gsvk_gsv* g) {
  if (!g) return;
  if (g->map) ::munmap(g->map, static_cast<size_t>(g->size));
  delete g;
}

extern "C" int gsvk_gsv_header(const gsvk_gsv* g, uint32_t* version, uint32_t* flags,
                               const char** name, size_t* name_len, const char** config_json,
                               size_t* config_len, uint32_t* n_tensors) {
  if (!g) return GSVK_E_NULL;
  if (version) *version = g->version;
  if (flags) *flags = g->flags;
  if (name) *name = g->name;
  if (name_len) *name_len = g->name_len;
  if (config_json) *config_json = g->config;
  if (config_len) *config_len = g->config_len;
  if (n_tensors) *n_tensors = g->n_tensors;
  return GSVK_OK;
}

extern "C" int gsvk_gsv_tensor_at(const gsvk_gsv* g, size_t index, gsvk_gsv_tensor* out) {
  if (!g || !out) return GSVK_E_NULL;
  if (index >= g->t.size()) return GSVK_E_SIZE;
  *out = g->t[index];
  return GSVK_OK;
}

extern "C" long gsvk_gsv_find(const gsvk_gsv* g, const char* name) {
  if (!g || !name) return -1;
  const size_t n = std::strlen(name);
  for (size_t i = 0; i < g->t.size(); ++i)
    if (g->t[i].name_len == n && std::memcmp(g->t[i].name, name, n) == 0)
      return static_cast<long>(i);
  return -1;
}

extern "C" int gsvk_gsv_arena(const gsvk_gsv* g, int kind, uint64_t* base, uint64_t* bytes) {
  if (!g || !base || !bytes) return GSVK_E_NULL;
  if (kind != GSVK_F16 && kind != GSVK_F32) return GSVK_E_DTYPE;
  uint64_t lo = UINT64_MAX, hi = 0;
  for (const auto& t : g->t) {
    uint64_t off, nb;
    if (!seg(t, kind, off, nb)) continue;
    lo = off < lo ? off : lo;
    hi = off + nb > hi ? off + nb : hi;
  }
  *base = hi ? lo : 0;
  *bytes = hi ? hi - lo : 0;
  return GSVK_OK;
}

extern "C" int gsvk_gsv_upload(const gsvk_gsv* g, int kind, void* device, size_t device_bytes,
                               void* stream) {
  uint64_t base = 0, bytes = 0;
  const int rc = gsvk_gsv_arena(g, kind, &base, &bytes);
  if (rc) return rc;
  if (!bytes) return GSVK_OK;
  if (!device) return GSVK_E_NULL;
  if (device_bytes < bytes) return GSVK_E_SIZE;
  // pageable (mapped) source: the runtime stages it through pinned buffers
  const hipError_t e = hipMemcpyAsync(device, g->base + base, bytes, hipMemcpyHostToDevice,
                                      static_cast<hipStream_t>(stream));
  return e == hipSuccess ? GSVK_OK : GSVK_E_HIP;
}

extern "C" const void* gsvk_gsv_device_ptr(const gsvk_gsv* g, int kind, const void* device,
                                           size_t index) {
  if (!g || !device || index >= g->t.size()) return nullptr;
  uint64_t base = 0, bytes = 0, off = 0, nb = 0;
  if (gsvk_gsv_arena(g, kind, &base, &bytes) || !seg(g->t[index], kind, off, nb)) return nullptr;
  return static_cast<const uint8_t*>(device) + (off - base);
}
