/*
 * mvlm_gguf.h -- GGUF reader and upload repacker of the MI355X matmul path.
 *
 * Replaces the reference's GGUF loader (src/models/gguf_loader.h:65-116,
 * gguf_loader.cpp:163-349) and the weight upload of the model
 * (upload_weight_image, src/models/moondream2.cpp:62-84).  The file is
 * memory-mapped read-only; tensor data and metadata strings are returned as
 * pointers into the mapping, valid until mvlm_gguf_close.  Differences from
 * the reference, on purpose:
 *  - the data section is aligned to the file's general.alignment (uint32
 *    metadata, default 32), which the reference hard-codes to 32
 *    (gguf_loader.cpp:332-337);
 *  - every tensor's byte range is checked against the file size;
 *  - mvlm_weight_from_gguf packs a tensor with GGUF dims (ne0 = K contiguous,
 *    ne1 = N) into the packed [N][K] HBM layout, for F32/F16/BF16/Q8_0/Q4_0.
 *    The reference uploaded F16 tensors with rows/cols swapped and passed
 *    quantized ones as raw buffers to image kernels (moondream2.cpp:62-84).
 * Status codes, error logging and mvlm_last_error() are those of mvlm_hip.h.
 */
#ifndef MVLM_GGUF_H
#define MVLM_GGUF_H

#include <stdint.h>

#include "mvlm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mvlm_gguf mvlm_gguf;

/* GGUF metadata value types (the GGUF specification; gguf_loader.h:33-38) */
enum mvlm_gguf_value_type {
    MVLM_GGUF_UINT8 = 0, MVLM_GGUF_INT8 = 1, MVLM_GGUF_UINT16 = 2, MVLM_GGUF_INT16 = 3,
    MVLM_GGUF_UINT32 = 4, MVLM_GGUF_INT32 = 5, MVLM_GGUF_FLOAT32 = 6, MVLM_GGUF_BOOL = 7,
    MVLM_GGUF_STRING = 8, MVLM_GGUF_ARRAY = 9, MVLM_GGUF_UINT64 = 10, MVLM_GGUF_INT64 = 11,
    MVLM_GGUF_FLOAT64 = 12
};

/* Header facts (GGUFHeader, gguf_loader.h:40-45, plus the resolved layout). */
typedef struct mvlm_gguf_info {
    uint32_t version;
    uint64_t tensor_count;
    uint64_t metadata_kv_count;
    uint64_t alignment;        /* general.alignment or 32 */
    uint64_t data_offset;      /* file offset of the tensor data section */
    uint64_t file_size;
} mvlm_gguf_info;

/* One tensor (TensorInfo, gguf_loader.h:52-59).  dims[i] = 1 for i >= n_dims. */
typedef struct mvlm_gguf_tensor {
    const char* name;          /* not NUL-terminated; name_len bytes */
    uint64_t name_len;
    uint32_t n_dims;
    uint64_t dims[4];
    uint32_t type;             /* ggml type id */
    uint64_t offset;           /* from the start of the data section */
    uint64_t bytes;            /* 0 for a type of unknown size */
} mvlm_gguf_tensor;

/* gguf_open (gguf_loader.cpp:163): map and parse; MVLM_ERR_FORMAT on a bad
 * magic, an unsupported version, truncation, > 4 dims, a tensor past the end. */
int mvlm_gguf_open(const char* path, mvlm_gguf** out);
/* gguf_close (gguf_loader.cpp:364) */
int mvlm_gguf_close(mvlm_gguf* g);
int mvlm_gguf_get_info(const mvlm_gguf* g, mvlm_gguf_info* out);
int mvlm_gguf_tensor_info(const mvlm_gguf* g, uint64_t index, mvlm_gguf_tensor* out);
/* gguf_find_tensor (gguf_loader.cpp:351): MVLM_ERR_NOT_FOUND if absent */
int mvlm_gguf_find_tensor(const mvlm_gguf* g, const char* name, uint64_t* index);
/* gguf_tensor_data (gguf_loader.cpp:360) */
int mvlm_gguf_tensor_data(const mvlm_gguf* g, uint64_t index, const void** data);

/* Metadata (gguf_loader.cpp:450-555).  get_u32 accepts UINT32 and INT32
 * values like the reference; get_array returns the element type, count and,
 * for fixed-size element types, a pointer to the packed elements (NULL for
 * string arrays, read with get_array_string). */
int mvlm_gguf_get_u32(const mvlm_gguf* g, const char* key, uint32_t* out);
int mvlm_gguf_get_string(const mvlm_gguf* g, const char* key, const char** str, uint64_t* len);
int mvlm_gguf_get_array(const mvlm_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count,
                        const void** data);
int mvlm_gguf_get_array_string(const mvlm_gguf* g, const char* key, uint64_t i, const char** str,
                               uint64_t* len);

/* ggml_type_size / ggml_type_block_size (gguf_loader.cpp:13-55): bytes per
 * block and elements per block of a ggml type; MVLM_ERR_NOT_FOUND if unknown. */
int mvlm_ggml_type_size(uint32_t type, uint64_t* block_bytes, uint32_t* block_elems);

/* upload_weight_image (moondream2.cpp:62-84) for the packed layout: a 2-D
 * tensor of type F32/F16/BF16/Q8_0/Q4_0 with ne0 = K, ne1 = N. */
int mvlm_weight_from_gguf(mvlm_device* dev, const mvlm_gguf* g, uint64_t index, mvlm_weight** out);

#ifdef __cplusplus
}
#endif

#endif /* MVLM_GGUF_H */
