/*
 * tc_gguf.h -- C-ABI GGUF v3 tensor reader of libtc_hip.so: opens a checkpoint,
 * lists its tensor records, and hands their raw block bytes to the mat-vec /
 * GEMM entry points (host pointer into a read-only mapping, or a copy into
 * device memory).
 *
 * Replaces the tensor side of tinycoder::GGUFLoader (include/GGUFLoader.hpp:48,
 * src/cpp/core/GGUFLoader.cpp): same file format, same record fields, the same
 * metadata string rendering. Every offset, count and length read from the file
 * is checked against the file size; a malformed file is refused with a
 * message (tc_last_error), never read out of bounds.
 */
#ifndef TC_GGUF_H
#define TC_GGUF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tc_gguf tc_gguf;

/* Parse the header, metadata and tensor records and map the tensor data
 * section read-only (GGUFLoader::load, GGUFLoader.cpp:212-240; the mapping is
 * file-backed like the reference's mapTensorData, :747). NULL on failure. */
tc_gguf *tc_gguf_open(const char *path);

/* Header, metadata and tensor records only; no mapping, tensor data pointers
 * are NULL (GGUFLoader::loadMetadata, GGUFLoader.cpp:163-190). */
tc_gguf *tc_gguf_open_metadata(const char *path);

void tc_gguf_close(tc_gguf *g);

/* GGUF header fields. */
uint32_t tc_gguf_version(const tc_gguf *g);
uint64_t tc_gguf_tensor_count(const tc_gguf *g);
uint64_t tc_gguf_metadata_count(const tc_gguf *g);
/* File offset of the tensor data section (the position after the records
 * rounded up to the alignment: 32, or general.alignment when present). */
uint64_t tc_gguf_data_offset(const tc_gguf *g);

/* Index of the tensor called `name`, or -1 (GGUFLoader::getTensorInfo,
 * GGUFLoader.cpp:1001-1015). */
int64_t tc_gguf_find_tensor(const tc_gguf *g, const char *name);

/* Record i (file order, as tensorRecords(), GGUFLoader.cpp:1020-1036): name
 * (valid until tc_gguf_close), GGML type id, dimension count (<= 4), dims in
 * file order (ne[0] = the contiguous row length), data offset relative to the
 * data section, and byte size (blocks x block bytes; 0 for an unknown type).
 * Any output pointer may be NULL. Returns TC_OK or TC_E_ARG. */
int tc_gguf_tensor_info(const tc_gguf *g, uint64_t i, const char **name, uint32_t *type, uint32_t *n_dims,
                        uint64_t *dims, uint64_t *offset, uint64_t *bytes);

/* Host pointer to tensor i's bytes inside the mapping (GGUFLoader::getTensor,
 * GGUFLoader.cpp:987-999), NULL for a metadata-only handle. */
const void *tc_gguf_tensor_data(const tc_gguf *g, uint64_t i);

/* Copy tensor i's bytes to device memory `dst` (dst_bytes >= its size) on
 * `stream` (hipStream_t as void*), and wait for the copy. */
int tc_gguf_upload(const tc_gguf *g, uint64_t i, void *dst, uint64_t dst_bytes, void *stream);

/* Metadata value of `key` rendered as the reference's metadata map holds it
 * (GGUFLoader.cpp:287-593): integers in decimal, floats as std::to_string
 * ("%f"), bools "true"/"false", strings verbatim, numeric arrays as their
 * first element (".rope.dimension_sections" arrays as all elements joined
 * with ","); string arrays and empty arrays have no entry. NULL if absent;
 * valid until tc_gguf_close. */
const char *tc_gguf_meta(const tc_gguf *g, const char *key);

/* GGML block geometry (ggmlTypeSize / ggmlBlockSize, GGUFLoader.cpp:64-160):
 * bytes per block and weights per block; 0 / 1 for unknown types. */
uint32_t tc_gguf_type_size(uint32_t type);
uint32_t tc_gguf_block_size(uint32_t type);

#ifdef __cplusplus
}
#endif
#endif
