// GGUF v3 directory reader (host only). Restates gguf.parseDiagnosed
// (inference/src/formats/gguf.zig:311-410) over a byte span: same limits,
// same validation order, same errors. Tensor weights are never read here;
// their byte ranges are validated. nuq_gguf_upload (api.hip) moves the data
// section to the device.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <string>
#include <string_view>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "gguf_doc.h"
#include "nuq_gguf.h"

namespace {

// gguf.retained_array_items / retained_key_prefixes / retained_prefixed_items
// (gguf.zig:41-47).
constexpr uint64_t kRetainedArrayItems = 64;
constexpr uint64_t kRetainedPrefixedItems = 65536;
constexpr const char *kRetainedPrefixes[] = {"prism.hadamard."};

struct Layout {
    uint64_t elements_per_block, bytes_per_block;
};

// encoding.layout (inference/src/tensor/encoding.zig:29-56): only the
// layouts the reference has checked are sized; any other id is refused.
bool layout_of(uint32_t id, Layout *l) {
    switch (id) {
        case 0: *l = {1, 4}; return true;        // F32
        case 1: *l = {1, 2}; return true;        // F16
        case 2: *l = {32, 18}; return true;      // Q4_0
        case 6: *l = {32, 22}; return true;      // Q5_0
        case 7: *l = {32, 24}; return true;      // Q5_1
        case 8: *l = {32, 34}; return true;      // Q8_0
        case 10: *l = {256, 84}; return true;    // Q2_K
        case 11: *l = {256, 110}; return true;   // Q3_K
        case 12: *l = {256, 144}; return true;   // Q4_K
        case 13: *l = {256, 176}; return true;   // Q5_K
        case 14: *l = {256, 210}; return true;   // Q6_K
        case 16: *l = {256, 66}; return true;    // IQ2_XXS
        case 17: *l = {256, 74}; return true;    // IQ2_XS
        case 18: *l = {256, 98}; return true;    // IQ3_XXS
        case 19: *l = {256, 50}; return true;    // IQ1_S
        case 20: *l = {32, 18}; return true;     // IQ4_NL
        case 21: *l = {256, 110}; return true;   // IQ3_S
        case 22: *l = {256, 82}; return true;    // IQ2_S
        case 23: *l = {256, 136}; return true;   // IQ4_XS
        case 29: *l = {256, 56}; return true;    // IQ1_M
        case 30: *l = {1, 2}; return true;       // BF16
        case 142: *l = {128, 34}; return true;   // PQ2_0
        case 143: *l = {128, 28}; return true;   // PTQ1_0
        default: return false;
    }
}

bool mul_overflows(uint64_t a, uint64_t b, uint64_t *out) { return __builtin_mul_overflow(a, b, out); }

// Layout.byteCount (encoding.zig:15-24).
int byte_count(const Layout &l, const uint64_t *dims, uint32_t rank, uint64_t *bytes) {
    if (rank == 0 || dims[0] == 0 || dims[0] % l.elements_per_block != 0) return NUQ_INVALID_SHAPE;
    uint64_t b;
    if (mul_overflows(dims[0] / l.elements_per_block, l.bytes_per_block, &b)) return NUQ_GGUF_OVERFLOW;
    for (uint32_t i = 1; i < rank; ++i) {
        if (dims[i] == 0) return NUQ_INVALID_SHAPE;
        if (mul_overflows(b, dims[i], &b)) return NUQ_GGUF_OVERFLOW;
    }
    *bytes = b;
    return NUQ_OK;
}

// std.unicode.utf8ValidateSlice: well-formed UTF-8, no overlong forms, no
// surrogate halves, nothing above U+10FFFF.
bool utf8_valid(const uint8_t *s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) {
            ++i;
            continue;
        }
        size_t len;
        uint32_t cp;
        if ((c & 0xe0) == 0xc0) {
            len = 2;
            cp = c & 0x1f;
        } else if ((c & 0xf0) == 0xe0) {
            len = 3;
            cp = c & 0x0f;
        } else if ((c & 0xf8) == 0xf0) {
            len = 4;
            cp = c & 0x07;
        } else {
            return false;
        }
        if (n - i < len) return false;
        for (size_t k = 1; k < len; ++k) {
            if ((s[i + k] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3f);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000)) return false;
        if (cp >= 0xd800 && cp <= 0xdfff) return false;
        if (cp > 0x10ffff) return false;
        i += len;
    }
    return true;
}

// validateName (gguf.zig:273-277)
int validate_name(const std::string &name) {
    if (name.empty() || name.size() > 65535 || !utf8_valid((const uint8_t *)name.data(), name.size()))
        return NUQ_GGUF_INVALID_NAME;
    for (unsigned char b : name)
        if (b < 0x20 || b == 0x7f) return NUQ_GGUF_INVALID_NAME;
    return NUQ_OK;
}

bool retained_key(const std::string &key) {
    for (const char *p : kRetainedPrefixes)
        if (key.compare(0, strlen(p), p) == 0) return true;
    return false;
}

#define NUQ_TRY(expr)                  \
    do {                               \
        const int rc_ = (expr);        \
        if (rc_ != NUQ_OK) return rc_; \
    } while (0)

// gguf.zig:174-266 Cursor. `position` counts bytes consumed; advance checks
// the claimed file length, then the directory limit; a read past the bytes
// actually present is EndOfStream, as for a reader that ends early.
struct Cursor {
    const uint8_t *bytes;
    uint64_t avail;
    uint64_t position = 0;
    uint64_t file_bytes;
    nuq_gguf_limits limits;

    int advance(uint64_t n) {
        if (position > file_bytes || n > file_bytes - position) return NUQ_GGUF_END_OF_STREAM;
        if (position > limits.directory_bytes || n > limits.directory_bytes - position) return NUQ_GGUF_LIMIT_EXCEEDED;
        position += n;
        return NUQ_OK;
    }
    // the bytes [position - n, position) just advanced over, if present
    int take(uint64_t n, const uint8_t **p) {
        const uint64_t start = position;
        NUQ_TRY(advance(n));
        if (position > avail) return NUQ_GGUF_END_OF_STREAM;
        *p = bytes + start;
        return NUQ_OK;
    }
    template <typename T>
    int integer(T *v) {
        const uint8_t *p;
        NUQ_TRY(take(sizeof(T), &p));
        memcpy(v, p, sizeof(T));  // little-endian host
        return NUQ_OK;
    }
    int skip(uint64_t n) {
        NUQ_TRY(advance(n));
        if (position > avail) return NUQ_GGUF_END_OF_STREAM;
        return NUQ_OK;
    }
    int string(std::string *out) {
        uint64_t len;
        NUQ_TRY(integer(&len));
        if (len > limits.string_bytes) return NUQ_GGUF_LIMIT_EXCEEDED;
        const uint8_t *p;
        NUQ_TRY(take(len, &p));
        out->assign((const char *)p, len);
        return NUQ_OK;
    }
    int kind(uint32_t *t) {
        NUQ_TRY(integer(t));
        return *t <= NUQ_GGUF_FLOAT64 ? (int)NUQ_OK : (int)NUQ_GGUF_INVALID_METADATA_TYPE;
    }
    int value(uint32_t tag, bool retain, nuq::GgufValue *v);
};

int Cursor::value(uint32_t tag, bool retain, nuq::GgufValue *v) {
    v->type = tag;
    switch (tag) {
#define NUQ_INT_CASE(TAG, T, KIND, FIELD) \
    case TAG: {                           \
        T x;                              \
        NUQ_TRY(integer(&x));             \
        v->kind = KIND;                   \
        v->FIELD = x;                     \
        return NUQ_OK;                    \
    }
        NUQ_INT_CASE(NUQ_GGUF_UINT8, uint8_t, NUQ_GGUF_VALUE_UNSIGNED, u)
        NUQ_INT_CASE(NUQ_GGUF_UINT16, uint16_t, NUQ_GGUF_VALUE_UNSIGNED, u)
        NUQ_INT_CASE(NUQ_GGUF_UINT32, uint32_t, NUQ_GGUF_VALUE_UNSIGNED, u)
        NUQ_INT_CASE(NUQ_GGUF_UINT64, uint64_t, NUQ_GGUF_VALUE_UNSIGNED, u)
        NUQ_INT_CASE(NUQ_GGUF_INT8, int8_t, NUQ_GGUF_VALUE_SIGNED, i)
        NUQ_INT_CASE(NUQ_GGUF_INT16, int16_t, NUQ_GGUF_VALUE_SIGNED, i)
        NUQ_INT_CASE(NUQ_GGUF_INT32, int32_t, NUQ_GGUF_VALUE_SIGNED, i)
        NUQ_INT_CASE(NUQ_GGUF_INT64, int64_t, NUQ_GGUF_VALUE_SIGNED, i)
#undef NUQ_INT_CASE
        case NUQ_GGUF_FLOAT32: {
            float x;
            NUQ_TRY(integer(&x));
            v->kind = NUQ_GGUF_VALUE_FLOAT;
            v->f = x;
            return NUQ_OK;
        }
        case NUQ_GGUF_FLOAT64: {
            double x;
            NUQ_TRY(integer(&x));
            v->kind = NUQ_GGUF_VALUE_FLOAT;
            v->f = x;
            return NUQ_OK;
        }
        case NUQ_GGUF_BOOLEAN: {
            uint8_t b;
            NUQ_TRY(integer(&b));
            if (b > 1) return NUQ_GGUF_INVALID_BOOLEAN;
            v->kind = NUQ_GGUF_VALUE_BOOLEAN;
            v->u = b;
            return NUQ_OK;
        }
        case NUQ_GGUF_STRING:
            v->kind = NUQ_GGUF_VALUE_STRING;
            return string(&v->str);
        case NUQ_GGUF_ARRAY: {
            uint32_t element;
            NUQ_TRY(kind(&element));
            if (element == NUQ_GGUF_ARRAY) return NUQ_GGUF_UNSUPPORTED_NESTED_ARRAY;
            uint64_t count;
            NUQ_TRY(integer(&count));
            if (count > limits.array_items) return NUQ_GGUF_LIMIT_EXCEEDED;
            v->kind = NUQ_GGUF_VALUE_ARRAY;
            v->element_type = element;
            v->count = count;
            v->file_offset = position;
            if (retain && count > kRetainedPrefixedItems) return NUQ_GGUF_LIMIT_EXCEEDED;
            if (retain || (element != NUQ_GGUF_STRING && count <= kRetainedArrayItems)) {
                v->values.resize(count);
                for (auto &item : v->values) NUQ_TRY(value(element, false, &item));
                v->retained = true;
            } else if (element == NUQ_GGUF_STRING) {
                for (uint64_t k = 0; k < count; ++k) {
                    uint64_t len;
                    NUQ_TRY(integer(&len));
                    if (len > limits.string_bytes) return NUQ_GGUF_LIMIT_EXCEEDED;
                    NUQ_TRY(skip(len));
                }
            } else if (element == NUQ_GGUF_BOOLEAN) {
                for (uint64_t k = 0; k < count; ++k) {
                    uint8_t b;
                    NUQ_TRY(integer(&b));
                    if (b > 1) return NUQ_GGUF_INVALID_BOOLEAN;
                }
            } else {
                uint64_t size = 0;
                switch (element) {
                    case NUQ_GGUF_UINT8: case NUQ_GGUF_INT8: size = 1; break;
                    case NUQ_GGUF_UINT16: case NUQ_GGUF_INT16: size = 2; break;
                    case NUQ_GGUF_UINT32: case NUQ_GGUF_INT32: case NUQ_GGUF_FLOAT32: size = 4; break;
                    default: size = 8; break;  // uint64, int64, float64
                }
                uint64_t total;
                if (mul_overflows(count, size, &total)) return NUQ_GGUF_OVERFLOW;
                NUQ_TRY(skip(total));
            }
            return NUQ_OK;
        }
        default:
            return NUQ_GGUF_INVALID_METADATA_TYPE;
    }
}

void note(nuq_gguf_rejection *r, const std::string &name, bool has_encoding, uint32_t encoding) {
    if (!r) return;
    r->len = (uint32_t)std::min<size_t>(name.size(), sizeof(r->tensor));
    memcpy(r->tensor, name.data(), r->len);
    r->has_encoding = has_encoding ? 1 : 0;
    r->encoding = has_encoding ? encoding : 0;
}

int parse_into(nuq_gguf *doc, const nuq_gguf_limits &limits, nuq_gguf_rejection *rejection) {
    Cursor c{doc->bytes, doc->avail, 0, doc->file_bytes, limits};
    uint32_t magic, version;
    NUQ_TRY(c.integer(&magic));
    if (magic != 0x46554747u) return NUQ_GGUF_INVALID_MAGIC;
    NUQ_TRY(c.integer(&version));
    if (version != 3) return NUQ_GGUF_UNSUPPORTED_VERSION;
    uint64_t tensor_count, metadata_count;
    NUQ_TRY(c.integer(&tensor_count));
    NUQ_TRY(c.integer(&metadata_count));
    if (tensor_count > limits.tensor_count || metadata_count > limits.metadata_count) return NUQ_GGUF_LIMIT_EXCEEDED;

    doc->metadata.resize(metadata_count);
    std::unordered_set<std::string_view> keys;
    uint32_t alignment = 32;
    for (auto &entry : doc->metadata) {
        NUQ_TRY(c.string(&entry.key));
        NUQ_TRY(validate_name(entry.key));
        if (!keys.insert(entry.key).second) return NUQ_GGUF_DUPLICATE_METADATA;
        uint32_t tag;
        NUQ_TRY(c.kind(&tag));
        NUQ_TRY(c.value(tag, retained_key(entry.key), &entry.value));
        if (entry.key == "general.alignment") {
            if (tag != NUQ_GGUF_UINT32) return NUQ_GGUF_INVALID_ALIGNMENT;
            alignment = (uint32_t)entry.value.u;
            if (alignment == 0 || (alignment & (alignment - 1)) != 0) return NUQ_GGUF_INVALID_ALIGNMENT;
        }
    }

    doc->tensors.resize(tensor_count);
    for (auto &t : doc->tensors) {
        NUQ_TRY(c.string(&t.name));
        NUQ_TRY(validate_name(t.name));
        if (!doc->tensor_index.emplace(t.name, (uint64_t)(&t - doc->tensors.data())).second)
            return NUQ_GGUF_DUPLICATE_TENSOR;
        NUQ_TRY(c.integer(&t.rank));
        if (t.rank == 0 || t.rank > 4) {
            note(rejection, t.name, false, 0);
            return NUQ_INVALID_SHAPE;
        }
        for (uint32_t i = 0; i < t.rank; ++i) NUQ_TRY(c.integer(&t.dims[i]));
        NUQ_TRY(c.integer(&t.encoding));
        // the shape is judged once the encoding is read, so a rejection names both
        uint64_t elements = 1;
        for (uint32_t i = 0; i < t.rank; ++i) {
            int rc = NUQ_OK;
            if (t.dims[i] == 0) rc = NUQ_INVALID_SHAPE;
            else if (mul_overflows(elements, t.dims[i], &elements)) rc = NUQ_GGUF_OVERFLOW;
            if (rc != NUQ_OK) {
                note(rejection, t.name, true, t.encoding);
                return rc;
            }
        }
        Layout l;
        if (!layout_of(t.encoding, &l)) {
            note(rejection, t.name, true, t.encoding);
            return NUQ_GGUF_UNSUPPORTED_TENSOR_TYPE;
        }
        const int rc = byte_count(l, t.dims, t.rank, &t.bytes);
        if (rc != NUQ_OK) {
            note(rejection, t.name, true, t.encoding);
            return rc;
        }
        NUQ_TRY(c.integer(&t.offset));
        if (t.offset % alignment != 0) return NUQ_GGUF_INVALID_ALIGNMENT;
        t.elements = elements;
    }

    const uint64_t padding = (alignment - c.position % alignment) % alignment;
    uint64_t data_offset;
    if (__builtin_add_overflow(c.position, padding, &data_offset)) return NUQ_GGUF_OVERFLOW;
    if (data_offset > doc->file_bytes) return NUQ_GGUF_END_OF_STREAM;
    // Descriptors need not be in offset order: check overlaps on a sorted copy.
    std::vector<std::pair<uint64_t, uint64_t>> ordered;
    ordered.reserve(doc->tensors.size());
    for (const auto &t : doc->tensors) ordered.emplace_back(t.offset, t.bytes);
    std::stable_sort(ordered.begin(), ordered.end(),
                     [](const auto &a, const auto &b) { return a.first < b.first; });
    uint64_t previous_end = 0;
    const uint64_t room = doc->file_bytes - data_offset;
    for (const auto &[offset, bytes] : ordered) {
        if (offset > room || bytes > room - offset) return NUQ_GGUF_TENSOR_OUT_OF_BOUNDS;
        if (offset < previous_end) return NUQ_GGUF_OVERLAPPING_TENSORS;
        previous_end = offset + bytes;
    }
    doc->version = version;
    doc->alignment = alignment;
    doc->directory_bytes = c.position;
    doc->data_offset = data_offset;
    return NUQ_OK;
}

void fill_value(const nuq::GgufValue &v, nuq_gguf_value *out) {
    memset(out, 0, sizeof(*out));
    out->kind = v.kind;
    out->type = v.type;
    out->u = v.u;
    out->i = v.i;
    out->f = v.f;
    if (v.kind == NUQ_GGUF_VALUE_STRING) {
        out->string = v.str.data();
        out->string_len = v.str.size();
    }
    if (v.kind == NUQ_GGUF_VALUE_ARRAY) {
        out->element_type = v.element_type;
        out->count = v.count;
        out->file_offset = v.file_offset;
        out->retained = v.retained ? v.values.size() : 0;
    }
}

int finish(nuq_gguf *doc, const nuq_gguf_limits *limits, nuq_gguf **out, nuq_gguf_rejection *rejection) {
    nuq_gguf_limits l;
    if (limits) l = *limits;
    else nuq_gguf_default_limits(&l);
    int rc;
    try {
        rc = parse_into(doc, l, rejection);
    } catch (const std::bad_alloc &) {
        rc = NUQ_GGUF_OUT_OF_MEMORY;
    }
    if (rc != NUQ_OK) {
        nuq_gguf_close(doc);
        return rc;
    }
    *out = doc;
    return NUQ_OK;
}

}  // namespace

extern "C" {

void nuq_gguf_default_limits(nuq_gguf_limits *l) {
    if (!l) return;
    l->directory_bytes = 64ull << 20;
    l->metadata_count = 16384;
    l->tensor_count = 100000;
    l->string_bytes = 1ull << 20;
    l->array_items = 4000000;
}

int nuq_gguf_parse(const void *bytes, uint64_t avail, uint64_t file_bytes, const nuq_gguf_limits *limits,
                   nuq_gguf **out, nuq_gguf_rejection *rejection) {
    if (!out || (!bytes && avail)) return NUQ_INVALID_ARGUMENT;
    *out = nullptr;
    nuq_gguf *doc = new (std::nothrow) nuq_gguf();
    if (!doc) return NUQ_GGUF_OUT_OF_MEMORY;
    doc->bytes = (const uint8_t *)bytes;
    doc->avail = std::min(avail, file_bytes);
    doc->file_bytes = file_bytes;
    return finish(doc, limits, out, rejection);
}

int nuq_gguf_open(const char *path, const nuq_gguf_limits *limits, nuq_gguf **out, nuq_gguf_rejection *rejection) {
    if (!out || !path) return NUQ_INVALID_ARGUMENT;
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return NUQ_GGUF_FILE_ERROR;
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return NUQ_GGUF_FILE_ERROR;
    }
    if (!S_ISREG(st.st_mode)) {
        close(fd);
        return NUQ_GGUF_NOT_REGULAR_FILE;
    }
    const uint64_t size = (uint64_t)st.st_size;
    if (size == 0 || size > (128ull << 30)) {
        close(fd);
        return NUQ_GGUF_LIMIT_EXCEEDED;
    }
    void *map = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);  // the mapping keeps the file
    if (map == MAP_FAILED) return NUQ_GGUF_FILE_ERROR;
    nuq_gguf *doc = new (std::nothrow) nuq_gguf();
    if (!doc) {
        munmap(map, size);
        return NUQ_GGUF_OUT_OF_MEMORY;
    }
    doc->map = map;
    doc->map_len = size;
    doc->bytes = (const uint8_t *)map;
    doc->avail = size;
    doc->file_bytes = size;
    return finish(doc, limits, out, rejection);
}

void nuq_gguf_close(nuq_gguf *g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->map_len);
    delete g;
}

int nuq_gguf_info_get(const nuq_gguf *g, nuq_gguf_info *info) {
    if (!g || !info) return NUQ_INVALID_ARGUMENT;
    info->version = g->version;
    info->alignment = g->alignment;
    info->file_bytes = g->file_bytes;
    info->directory_bytes = g->directory_bytes;
    info->data_offset = g->data_offset;
    info->metadata_count = g->metadata.size();
    info->tensor_count = g->tensors.size();
    return NUQ_OK;
}

int nuq_gguf_metadata(const nuq_gguf *g, uint64_t index, const char **key, uint64_t *key_len, nuq_gguf_value *value) {
    if (!g || !key || !key_len || !value) return NUQ_INVALID_ARGUMENT;
    if (index >= g->metadata.size()) return NUQ_GGUF_NOT_FOUND;
    const auto &m = g->metadata[index];
    *key = m.key.data();
    *key_len = m.key.size();
    fill_value(m.value, value);
    return NUQ_OK;
}

int nuq_gguf_get(const nuq_gguf *g, const char *key, uint64_t key_len, nuq_gguf_value *value) {
    if (!g || (!key && key_len) || !value) return NUQ_INVALID_ARGUMENT;
    const std::string_view want(key ? key : "", key_len);
    for (const auto &m : g->metadata)
        if (m.key == want) {
            fill_value(m.value, value);
            return NUQ_OK;
        }
    return NUQ_GGUF_NOT_FOUND;
}

int nuq_gguf_array_value(const nuq_gguf *g, uint64_t index, uint64_t item, nuq_gguf_value *value) {
    if (!g || !value) return NUQ_INVALID_ARGUMENT;
    if (index >= g->metadata.size()) return NUQ_GGUF_NOT_FOUND;
    const auto &v = g->metadata[index].value;
    if (v.kind != NUQ_GGUF_VALUE_ARRAY || !v.retained || item >= v.values.size()) return NUQ_GGUF_NOT_FOUND;
    fill_value(v.values[item], value);
    return NUQ_OK;
}

int nuq_gguf_tensor_get(const nuq_gguf *g, uint64_t index, nuq_gguf_tensor *out) {
    if (!g || !out) return NUQ_INVALID_ARGUMENT;
    if (index >= g->tensors.size()) return NUQ_GGUF_NOT_FOUND;
    const auto &t = g->tensors[index];
    memset(out, 0, sizeof(*out));
    out->name = t.name.data();
    out->name_len = t.name.size();
    out->rank = t.rank;
    out->encoding = t.encoding;
    for (uint32_t i = 0; i < t.rank; ++i) out->dimensions[i] = t.dims[i];
    out->offset = t.offset;
    out->bytes = t.bytes;
    out->elements = t.elements;
    return NUQ_OK;
}

int nuq_gguf_find_tensor(const nuq_gguf *g, const char *name, uint64_t name_len, uint64_t *index) {
    if (!g || (!name && name_len) || !index) return NUQ_INVALID_ARGUMENT;
    const auto it = g->tensor_index.find(std::string_view(name ? name : "", name_len));
    if (it == g->tensor_index.end()) return NUQ_GGUF_NOT_FOUND;
    *index = it->second;
    return NUQ_OK;
}

int nuq_gguf_directory(const nuq_gguf *g, const void **bytes, uint64_t *len) {
    if (!g || !bytes || !len) return NUQ_INVALID_ARGUMENT;
    *bytes = g->bytes;
    *len = std::min(g->directory_bytes, g->avail);
    return NUQ_OK;
}

// ArrayReader (gguf.zig:63-104)
int nuq_gguf_array_reader_init(nuq_gguf_array_reader *r, uint32_t element_type, uint64_t count, uint64_t file_offset,
                               const void *directory, uint64_t directory_len, const nuq_gguf_limits *limits) {
    if (!r || (!directory && directory_len)) return NUQ_INVALID_ARGUMENT;
    nuq_gguf_limits l;
    if (limits) l = *limits;
    else nuq_gguf_default_limits(&l);
    if (directory_len > l.directory_bytes || count > l.array_items) return NUQ_GGUF_LIMIT_EXCEEDED;
    if (element_type != NUQ_GGUF_STRING && element_type != NUQ_GGUF_INT32) return NUQ_GGUF_INVALID_METADATA_TYPE;
    if (file_offset > directory_len) return NUQ_GGUF_END_OF_STREAM;
    const uint64_t len = directory_len - file_offset;
    const uint64_t minimum = element_type == NUQ_GGUF_STRING ? 8 : 4;
    if (count > len / minimum) return NUQ_GGUF_END_OF_STREAM;
    r->bytes = (const uint8_t *)directory + file_offset;
    r->len = len;
    r->remaining = count;
    r->kind = element_type;
    r->reserved = 0;
    r->string_bytes = l.string_bytes;
    return NUQ_OK;
}

int nuq_gguf_array_next_string(nuq_gguf_array_reader *r, const char **value, uint64_t *len, int *has) {
    if (!r || !value || !len || !has) return NUQ_INVALID_ARGUMENT;
    *has = 0;
    if (r->kind != NUQ_GGUF_STRING) return NUQ_GGUF_INVALID_METADATA_TYPE;
    if (r->remaining == 0) return NUQ_OK;
    if (r->len < 8) return NUQ_GGUF_END_OF_STREAM;
    uint64_t n;
    memcpy(&n, r->bytes, 8);
    if (n > r->string_bytes) return NUQ_GGUF_LIMIT_EXCEEDED;
    if (n > r->len - 8) return NUQ_GGUF_END_OF_STREAM;
    *value = (const char *)r->bytes + 8;
    *len = n;
    *has = 1;
    r->bytes += 8 + n;
    r->len -= 8 + n;
    r->remaining -= 1;
    return NUQ_OK;
}

int nuq_gguf_array_next_int32(nuq_gguf_array_reader *r, int32_t *value, int *has) {
    if (!r || !value || !has) return NUQ_INVALID_ARGUMENT;
    *has = 0;
    if (r->kind != NUQ_GGUF_INT32) return NUQ_GGUF_INVALID_METADATA_TYPE;
    if (r->remaining == 0) return NUQ_OK;
    if (r->len < 4) return NUQ_GGUF_END_OF_STREAM;
    memcpy(value, r->bytes, 4);
    *has = 1;
    r->bytes += 4;
    r->len -= 4;
    r->remaining -= 1;
    return NUQ_OK;
}

// View.bytes (runtime/weights.zig:11-15)
int nuq_gguf_tensor_bytes(const nuq_gguf *g, uint64_t index, const void **bytes, uint64_t *len) {
    if (!g || !bytes || !len) return NUQ_INVALID_ARGUMENT;
    if (index >= g->tensors.size()) return NUQ_GGUF_NOT_FOUND;
    const auto &t = g->tensors[index];
    uint64_t start;
    if (__builtin_add_overflow(g->data_offset, t.offset, &start)) return NUQ_GGUF_OVERFLOW;
    if (start > g->avail || t.bytes > g->avail - start) return NUQ_GGUF_TENSOR_OUT_OF_BOUNDS;
    *bytes = g->bytes + start;
    *len = t.bytes;
    return NUQ_OK;
}

// View.matrix (runtime/weights.zig:16-19): columns = dims[0], rows = dims[1].
int nuq_gguf_matrix(const nuq_gguf *g, uint64_t index, const void *device_base, nuq_matrix *m) {
    if (!g || !m) return NUQ_INVALID_ARGUMENT;
    if (index >= g->tensors.size()) return NUQ_GGUF_NOT_FOUND;
    const auto &t = g->tensors[index];
    if (t.rank != 2) return NUQ_INVALID_SHAPE;
    const void *bytes;
    uint64_t len;
    if (device_base) {
        // the parse bounded offset + bytes by the data section
        bytes = (const uint8_t *)device_base + t.offset;
        len = t.bytes;
    } else {
        NUQ_TRY(nuq_gguf_tensor_bytes(g, index, &bytes, &len));
    }
    m->encoding = t.encoding;
    m->reserved = 0;
    m->columns = t.dims[0];
    m->rows = t.dims[1];
    m->bytes = bytes;
    m->byte_len = len;
    return NUQ_OK;
}

uint64_t nuq_gguf_data_bytes(const nuq_gguf *g) { return g ? g->file_bytes - g->data_offset : 0; }

}  // extern "C"
