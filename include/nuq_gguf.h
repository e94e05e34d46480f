/*
 * nuq_gguf — GGUF v3 directory reader and device upload for libnuq.
 *
 * Replaces the loading half of nuclis's weight path:
 *  - nuq_gguf_parse / nuq_gguf_open restate gguf.parse / gguf.parseDiagnosed
 *    (inference/src/formats/gguf.zig:311-410) and weights.Mapped.open
 *    (runtime/weights.zig:63-78): the header, metadata and tensor
 *    descriptors are read and validated with the same limits, in the same
 *    order, to the same errors; no tensor weights are read.
 *  - nuq_gguf_upload copies the file's tensor-data section, unchanged, into
 *    one caller-owned device allocation. Every tensor keeps its offset, so a
 *    device matrix is `base + tensor.offset` (nuq_gguf_matrix, the device
 *    twin of weights.View.matrix, runtime/weights.zig:16-19). GGUF aligns
 *    tensors to `general.alignment` (32 by default), which covers the 16-byte
 *    alignment the vector kernels want for Q4_K / Q5_K rows.
 *
 * Status codes are the nuq_status values of nuq.h; the GGUF errors carry
 * the names of gguf.Error (gguf.zig:156-172) beside them.
 */
#ifndef NUQ_GGUF_H
#define NUQ_GGUF_H

#include "nuq.h"

#ifdef __cplusplus
extern "C" {
#endif

/* gguf.Error names beyond those nuq.h already has (InvalidShape = 1). */
enum nuq_gguf_status {
    NUQ_GGUF_END_OF_STREAM = 20,          /* error.EndOfStream */
    NUQ_GGUF_INVALID_MAGIC = 21,          /* error.InvalidMagic */
    NUQ_GGUF_UNSUPPORTED_VERSION = 22,    /* error.UnsupportedVersion */
    NUQ_GGUF_LIMIT_EXCEEDED = 23,         /* error.LimitExceeded */
    NUQ_GGUF_INVALID_METADATA_TYPE = 24,  /* error.InvalidMetadataType */
    NUQ_GGUF_UNSUPPORTED_NESTED_ARRAY = 25, /* error.UnsupportedNestedArray */
    NUQ_GGUF_INVALID_BOOLEAN = 26,        /* error.InvalidBoolean */
    NUQ_GGUF_INVALID_NAME = 27,           /* error.InvalidName */
    NUQ_GGUF_DUPLICATE_METADATA = 28,     /* error.DuplicateMetadata */
    NUQ_GGUF_DUPLICATE_TENSOR = 29,       /* error.DuplicateTensor */
    NUQ_GGUF_INVALID_ALIGNMENT = 30,      /* error.InvalidAlignment */
    NUQ_GGUF_OVERFLOW = 31,               /* error.Overflow */
    NUQ_GGUF_UNSUPPORTED_TENSOR_TYPE = 32, /* error.UnsupportedTensorType */
    NUQ_GGUF_TENSOR_OUT_OF_BOUNDS = 33,   /* error.TensorOutOfBounds */
    NUQ_GGUF_OVERLAPPING_TENSORS = 34,    /* error.OverlappingTensors */
    NUQ_GGUF_OUT_OF_MEMORY = 35,          /* error.OutOfMemory */
    NUQ_GGUF_NOT_REGULAR_FILE = 36,       /* error.NotRegularFile */
    NUQ_GGUF_FILE_ERROR = 37,             /* open / stat / mmap failed */
    NUQ_GGUF_NOT_FOUND = 38               /* no such key or tensor (the reference returns null) */
};

/* gguf.Type (gguf.zig:21-35). */
enum nuq_gguf_type {
    NUQ_GGUF_UINT8 = 0, NUQ_GGUF_INT8 = 1, NUQ_GGUF_UINT16 = 2, NUQ_GGUF_INT16 = 3,
    NUQ_GGUF_UINT32 = 4, NUQ_GGUF_INT32 = 5, NUQ_GGUF_FLOAT32 = 6, NUQ_GGUF_BOOLEAN = 7,
    NUQ_GGUF_STRING = 8, NUQ_GGUF_ARRAY = 9, NUQ_GGUF_UINT64 = 10, NUQ_GGUF_INT64 = 11,
    NUQ_GGUF_FLOAT64 = 12
};

/* gguf.Value's active field (gguf.zig:105-112). */
enum nuq_gguf_value_kind {
    NUQ_GGUF_VALUE_UNSIGNED = 0, NUQ_GGUF_VALUE_SIGNED = 1, NUQ_GGUF_VALUE_FLOAT = 2,
    NUQ_GGUF_VALUE_BOOLEAN = 3, NUQ_GGUF_VALUE_STRING = 4, NUQ_GGUF_VALUE_ARRAY = 5
};

/* gguf.Limits (gguf.zig:13-19); nuq_gguf_default_limits fills the defaults. */
typedef struct nuq_gguf_limits {
    uint64_t directory_bytes;
    uint64_t metadata_count;
    uint64_t tensor_count;
    uint64_t string_bytes;
    uint64_t array_items;
} nuq_gguf_limits;

/* gguf.Value plus gguf.Array (gguf.zig:49-57). Strings point into the
 * document and are not NUL-terminated. `retained` is the number of values an
 * array keeps (0 for a lazy array: read it with nuq_gguf_array_reader). */
typedef struct nuq_gguf_value {
    uint32_t kind; /* nuq_gguf_value_kind */
    uint32_t type; /* nuq_gguf_type of the value as stored */
    uint64_t u;    /* UNSIGNED, BOOLEAN (0/1) */
    int64_t i;     /* SIGNED */
    double f;      /* FLOAT (float32 values widened) */
    const char *string;
    uint64_t string_len;
    uint32_t element_type; /* ARRAY */
    uint32_t reserved;
    uint64_t count;
    uint64_t file_offset;
    uint64_t retained;
} nuq_gguf_value;

/* gguf.Tensor (gguf.zig:114-122); `offset` is relative to data_offset. */
typedef struct nuq_gguf_tensor {
    const char *name;
    uint64_t name_len;
    uint32_t rank;
    uint32_t encoding;
    uint64_t dimensions[4];
    uint64_t offset;
    uint64_t bytes;
    uint64_t elements;
} nuq_gguf_tensor;

/* gguf.Document's scalars (gguf.zig:124-131). */
typedef struct nuq_gguf_info {
    uint32_t version;
    uint32_t alignment;
    uint64_t file_bytes;
    uint64_t directory_bytes;
    uint64_t data_offset;
    uint64_t metadata_count;
    uint64_t tensor_count;
} nuq_gguf_info;

/* gguf.Rejection (gguf.zig:287-301): the tensor behind an UnsupportedTensorType,
 * InvalidShape or Overflow rejection, its name truncated to 128 bytes.
 * has_encoding is 0 when the rank was refused before the encoding was read. */
typedef struct nuq_gguf_rejection {
    char tensor[128];
    uint32_t len;
    uint32_t has_encoding;
    uint32_t encoding;
    uint32_t reserved;
} nuq_gguf_rejection;

/* gguf.ArrayReader (gguf.zig:63-104): bounded sequential access to a lazy
 * string or int32 array in a borrowed directory image. */
typedef struct nuq_gguf_array_reader {
    const uint8_t *bytes;
    uint64_t len;
    uint64_t remaining;
    uint32_t kind;
    uint32_t reserved;
    uint64_t string_bytes;
} nuq_gguf_array_reader;

typedef struct nuq_gguf nuq_gguf;

void nuq_gguf_default_limits(nuq_gguf_limits *limits);

/* gguf.parseDiagnosed (gguf.zig:311-410) over `avail` bytes of a file that
 * is `file_bytes` long (the bytes past `avail` are missing, as for a reader
 * that ends early). limits and rejection may be NULL (defaults / not asked).
 * The document borrows `bytes`, which must outlive it; *out is NULL on error. */
int nuq_gguf_parse(const void *bytes, uint64_t avail, uint64_t file_bytes, const nuq_gguf_limits *limits,
                   nuq_gguf **out, nuq_gguf_rejection *rejection);
/* weights.Mapped.open (runtime/weights.zig:63-78): maps `path` read-only and
 * parses it; files of 0 bytes or above 128 GiB are LimitExceeded. */
int nuq_gguf_open(const char *path, const nuq_gguf_limits *limits, nuq_gguf **out, nuq_gguf_rejection *rejection);
/* Document.deinit / Mapped.deinit. */
void nuq_gguf_close(nuq_gguf *g);

int nuq_gguf_info_get(const nuq_gguf *g, nuq_gguf_info *info);
/* Metadata entry `index` in file order: its key (not NUL-terminated) and value. */
int nuq_gguf_metadata(const nuq_gguf *g, uint64_t index, const char **key, uint64_t *key_len, nuq_gguf_value *value);
/* Document.get (gguf.zig:141-146): NOT_FOUND when absent. */
int nuq_gguf_get(const nuq_gguf *g, const char *key, uint64_t key_len, nuq_gguf_value *value);
/* Value `item` of a retained array (metadata entry `index`). */
int nuq_gguf_array_value(const nuq_gguf *g, uint64_t index, uint64_t item, nuq_gguf_value *value);
/* Tensor descriptor `index` in file order. */
int nuq_gguf_tensor_get(const nuq_gguf *g, uint64_t index, nuq_gguf_tensor *tensor);
/* The tensor named `name`: its index (NOT_FOUND when absent). */
int nuq_gguf_find_tensor(const nuq_gguf *g, const char *name, uint64_t name_len, uint64_t *index);
/* The directory image [0, directory_bytes) for nuq_gguf_array_reader_init. */
int nuq_gguf_directory(const nuq_gguf *g, const void **bytes, uint64_t *len);

/* ArrayReader.init / nextString / nextInt32. `has` is 0 at the end. */
int nuq_gguf_array_reader_init(nuq_gguf_array_reader *r, uint32_t element_type, uint64_t count, uint64_t file_offset,
                               const void *directory, uint64_t directory_len, const nuq_gguf_limits *limits);
int nuq_gguf_array_next_string(nuq_gguf_array_reader *r, const char **value, uint64_t *len, int *has);
int nuq_gguf_array_next_int32(nuq_gguf_array_reader *r, int32_t *value, int *has);

/* weights.View.bytes (runtime/weights.zig:11-15): the host bytes of tensor
 * `index`, TensorOutOfBounds / Overflow as there. */
int nuq_gguf_tensor_bytes(const nuq_gguf *g, uint64_t index, const void **bytes, uint64_t *len);
/* weights.View.matrix (runtime/weights.zig:16-19) over a device image: a
 * rank-2 tensor as a nuq_matrix whose bytes are `device_base + offset`
 * (device_base NULL: the host mapping). InvalidShape for other ranks. */
int nuq_gguf_matrix(const nuq_gguf *g, uint64_t index, const void *device_base, nuq_matrix *matrix);

/* Size of the tensor-data section, [data_offset, file_bytes): the device
 * allocation nuq_gguf_upload fills. */
uint64_t nuq_gguf_data_bytes(const nuq_gguf *g);
/* Copies the tensor-data section to `device` (caller-owned, at least
 * nuq_gguf_data_bytes bytes) through pinned staging buffers on the
 * context's stream, and returns when the copy is complete. The section must
 * be fully present (avail == file_bytes). */
int nuq_gguf_upload(nuq_context *ctx, const nuq_gguf *g, void *device, uint64_t device_len);

#ifdef __cplusplus
}
#endif
#endif
