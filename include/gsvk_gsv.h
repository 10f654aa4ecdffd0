/*
 * gsvk_gsv.h — C ABI of the .gsv (GSV1) weight-container loader: open and validate a file, list its
 * tensors, and upload its fp16 or fp32 data segments to the GPU as one device arena each.
 *
 * Format (the reference's tools/convert.py docstring, read by src/runtime/gsv_header.cpp and
 * gsv_loader.cpp), little-endian:
 *   '<4s' magic "GSV1" | '<I' version = 1 | '<I' flags (bit0: some tensor has an fp16 segment)
 *   '<H' name length + UTF-8 name | '<I' config length + JSON | '<I' n_tensors
 *   n_tensors directory entries: '<H' name length + name | '<H' rank + rank x '<I' dims |
 *     '<H' source dtype (1 fp32, 2 fp16) | '<Q' f32 offset '<Q' f32 bytes | '<Q' f16 offset
 *     '<Q' f16 bytes (0: no fp16 copy)
 *   data: all fp32 segments, then all fp16 segments, each starting on a 64-byte boundary.
 * Because the fp16 segments are contiguous in the file, gsvk_gsv_upload moves all of them in one
 * host-to-device copy; a tensor's device address is then arena + (segment offset - arena base).
 *
 * Status: GSVK_OK, GSVK_E_NULL, GSVK_E_IO (cannot open / map), GSVK_E_FORMAT (the file breaks a
 * rule the reference's loader checks: magic, version, truncation, rank <= 8, dtype enum, segment
 * sizes against the shape, 64-byte alignment, segments inside the file, flags bit0 against the
 * directory), GSVK_E_SIZE (arena too small), GSVK_E_HIP (copy failed).
 */
#ifndef GSVK_GSV_H
#define GSVK_GSV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct gsvk_gsv gsvk_gsv;

typedef struct gsvk_gsv_tensor {
  const char* name; /* not NUL-terminated: name_len bytes inside the mapped file */
  size_t name_len;
  uint32_t rank;
  uint32_t dims[8];
  uint64_t numel;
  int src_dtype; /* 1 = fp32 source, 2 = fp16 source (the file's enum) */
  uint64_t f32_offset, f32_nbytes; /* f32_nbytes 0: slim file, fp16 copy only */
  uint64_t f16_offset, f16_nbytes; /* f16_nbytes 0: no fp16 copy (small tensors) */
} gsvk_gsv_tensor;

/* Map `path` read-only and validate header and directory (GsvFile::GsvFile, gsv_loader.cpp:112-150;
 * parse_gsv_raw_header, gsv_header.cpp:29-56; parse_gsv_directory, gsv_loader.cpp:46-108). */
int gsvk_gsv_open(const char* path, gsvk_gsv** out);
/* The same over a caller-owned buffer that outlives the handle (no copy). */
int gsvk_gsv_open_memory(const void* data, size_t size, gsvk_gsv** out);
void gsvk_gsv_close(gsvk_gsv* g);

/* Header fields; the name and the config JSON point into the file (not NUL-terminated). */
int gsvk_gsv_header(const gsvk_gsv* g, uint32_t* version, uint32_t* flags, const char** name,
                    size_t* name_len, const char** config_json, size_t* config_len,
                    uint32_t* n_tensors);
int gsvk_gsv_tensor_at(const gsvk_gsv* g, size_t index, gsvk_gsv_tensor* out);
/* Index of the tensor called `name` (NUL-terminated), or -1 (GsvFile::tensor). */
long gsvk_gsv_find(const gsvk_gsv* g, const char* name);

/* The file range [base, base + bytes) that holds every segment of one kind (kind = GSVK_F16: fp16
 * segments, GSVK_F32: fp32 segments); bytes = 0 when the file has none. */
int gsvk_gsv_arena(const gsvk_gsv* g, int kind, uint64_t* base, uint64_t* bytes);
/* Copy that range to device memory (at least `bytes`, 64-byte aligned recommended) on `stream`. */
int gsvk_gsv_upload(const gsvk_gsv* g, int kind, void* device, size_t device_bytes, void* stream);
/* Device address of tensor `index`'s segment of `kind` inside an arena uploaded to `device`, or
 * NULL when the tensor has no such segment. */
const void* gsvk_gsv_device_ptr(const gsvk_gsv* g, int kind, const void* device, size_t index);

#ifdef __cplusplus
}
#endif

#endif /* GSVK_GSV_H */
