/* .xinfer artifact access for the INT4 projection path: CRC-64, the container
 * reader and device upload of `<name>` / `<name>.scales` weight sections.
 *
 * Replaces, for a HIP device, the reference's artifact layer:
 *   src/artifact/container.h:11-63  (file layout: header, sections, footer)
 *   src/artifact/checksum.h:9-21    (CRC-64/ECMA-182, reflected)
 *   src/artifact/c_api.h:14-18      (xinfer_crc64, xinfer_crc64_file)
 *   src/artifact/reader.h:12-61     (ArtifactReader)
 *   src/targets/qwen3_8_27b/weights.cpp:252-303 (load_linear: read the weight
 *                                    and scale sections, size-check, upload)
 * Section payloads are verified on the GPU after the upload (a parallel
 * CRC-64 over device memory) instead of by a byte loop on the host.
 *
 * Status codes are those of xinfer_ops.h plus XINFER_ERR_IO and
 * XINFER_ERR_CHECKSUM below. */
#ifndef XINFER_HIP_ARTIFACT_H
#define XINFER_HIP_ARTIFACT_H

#include <stddef.h>
#include <stdint.h>

#include "xinfer_ops.h"

#ifdef __cplusplus
extern "C" {
#endif

#define XINFER_ERR_IO (-6)       /* file missing, short read, malformed container */
#define XINFER_ERR_CHECKSUM (-7) /* CRC-64 of a section or of the file differs */

/* ---------------------------------------------------------------- CRC-64 --
 * CRC-64/ECMA-182 in reflected form (polynomial 0xC96C5795D7870F42, register
 * initialised to all ones, result XORed with all ones): the checksum of
 * src/artifact/checksum.cpp:10-54.  "123456789" -> 0x995DC9BBDF1939FA. */

/* Replaces `xinfer_crc64` -- src/artifact/c_api.h:15, c_api.cpp:9-12
 * (0 for a null pointer or zero length, as there). */
uint64_t xinfer_crc64(const void* data, size_t length);

/* Replaces `xinfer_crc64_file` -- src/artifact/c_api.h:18, c_api.cpp:14-38:
 * CRC-64 of the first max_bytes bytes of a file (0 = whole file); 0 when the
 * file cannot be opened. */
uint64_t xinfer_crc64_file(const char* filepath, uint64_t max_bytes);

/* No reference counterpart (the reference checksums on the host only):
 * CRC-64 of `length` bytes of device memory, asynchronous on `stream`; the
 * result is written to *d_crc (device memory, 8-byte aligned).  `scratch` is
 * caller-owned device memory of xinfer_crc64_device_scratch_bytes(length)
 * bytes (NULL: a library buffer grown on first use). */
size_t xinfer_crc64_device_scratch_bytes(size_t length);
int xinfer_crc64_device(void* stream, const void* d_data, size_t length, uint64_t* d_crc,
                        void* scratch, size_t scratch_bytes);

/* ------------------------------------------------------------- container --
 * Same field order and sizes as FileHeader / SectionEntry / FileFooter
 * (src/artifact/container.h:35-63, packed little-endian). */
typedef struct xinfer_file_header {
    uint8_t magic[8]; /* "XINFER\0\0" */
    uint32_t format_version;
    uint32_t header_size;
    uint32_t flags;
    uint32_t section_count;
    uint64_t metadata_offset;
    uint64_t metadata_size;
    uint64_t section_table_offset;
    uint64_t section_table_size;
    uint64_t total_file_size;
} xinfer_file_header;

typedef struct xinfer_section_info {
    char name[96];
    uint32_t type_tag; /* SectionType, container.h:19-27 */
    uint32_t flags;
    uint64_t offset;
    uint64_t size;
    uint64_t checksum;
} xinfer_section_info;

typedef struct xinfer_artifact xinfer_artifact;

/* Replaces `ArtifactReader::open` -- src/artifact/reader.h:25, reader.cpp:56-196:
 * the same checks (magic, version, header size, file size, footer magic,
 * metadata and section bounds) in the same order.  On failure returns
 * XINFER_ERR_IO and, if err is non-NULL, a message (truncated to err_len). */
int xinfer_artifact_open(const char* filepath, xinfer_artifact** out, char* err, size_t err_len);

/* Replaces `ArtifactReader::close` -- reader.h:26.  Frees the reader's host
 * and device staging buffers; NULL is ignored. */
void xinfer_artifact_close(xinfer_artifact* a);

/* Replaces `header()`, `footer()` -- reader.h:30-31. */
int xinfer_artifact_header(const xinfer_artifact* a, xinfer_file_header* out);
int xinfer_artifact_footer(const xinfer_artifact* a, uint64_t* file_checksum);

/* Replaces `raw_metadata_json()` -- reader.h:36: the metadata block (not
 * NUL-terminated) and its length. */
const char* xinfer_artifact_metadata_json(const xinfer_artifact* a, size_t* length);

/* Replaces `list_sections()` / `get_section_info()` / `has_section()` --
 * reader.h:39-41.  _section_by_name returns XINFER_ERR_INVALID_ARG when the
 * section does not exist. */
int32_t xinfer_artifact_section_count(const xinfer_artifact* a);
int xinfer_artifact_section_at(const xinfer_artifact* a, int32_t index, xinfer_section_info* out);
int xinfer_artifact_section_by_name(const xinfer_artifact* a, const char* name, xinfer_section_info* out);

/* Replaces `read_section(name, dst, size)` -- reader.h:47, reader.cpp:240-276:
 * host buffer of at least the section size; CRC-64 checked against the
 * section table (XINFER_ERR_CHECKSUM on mismatch). */
int xinfer_artifact_read_section(xinfer_artifact* a, const char* name, void* dst, size_t dst_bytes,
                                 char* err, size_t err_len);

/* Replaces `validate_checksum()` -- reader.h:50, reader.cpp:278-318: CRC-64 of
 * every byte before the footer against the footer (host threads). */
int xinfer_artifact_validate_checksum(xinfer_artifact* a, char* err, size_t err_len);

/* No reference counterpart as one call (the reference reads to a host vector,
 * then copies; weights.cpp:268-293): read a section straight into device
 * memory through pinned, double-buffered staging on `stream`, and, when
 * verify != 0, check its CRC-64 on the GPU.  Returns once the data is on the
 * device (the stream is synchronised). */
int xinfer_artifact_upload_section(xinfer_artifact* a, const char* name, void* stream, void* d_dst,
                                   size_t dst_bytes, int verify, char* err, size_t err_len);

/* Replaces the `load_linear` helper of weights.cpp:252-303: sections `name`
 * ([out_features][in_features/2] packed INT4) and `name + ".scales"`
 * ([out_features][in_features/group_size] fp16), sizes checked exactly as
 * there, uploaded into new device allocations (hipMalloc; release with
 * hipFree) and CRC-verified on the GPU.  Fields as LinearWeightView,
 * weights.h:13-23. */
typedef struct xinfer_linear_weight_view {
    void* d_weights_int4;
    void* d_scales;
    int64_t in_features;
    int64_t out_features;
    int32_t group_size;
} xinfer_linear_weight_view;

int xinfer_artifact_load_linear(xinfer_artifact* a, const char* weight_name, int64_t out_features,
                                int64_t in_features, int32_t group_size, void* stream,
                                xinfer_linear_weight_view* out, char* err, size_t err_len);

#ifdef __cplusplus
}
#endif

#endif /* XINFER_HIP_ARTIFACT_H */
