/*
 * The GGUF directory reader (nuclis_amd/csrc/gguf.cpp, host code) under
 * AddressSanitizer and UndefinedBehaviorSanitizer, over the corruption
 * families of the reference's fuzz test (inference/src/formats/gguf.zig:
 * 617-650): every truncation at three claimed lengths, five byte values,
 * three u32 and five u64 values at every offset, and 200000 seeded random
 * edits of the reference's wire fixture (gguf.zig:424-471). Each parse must
 * return a status or a document; every document is walked (metadata, arrays,
 * lazy arrays through the reader, tensors, views) and closed. A read out of
 * bounds, a leak or undefined behaviour aborts the run. Prints
 * "gguf_fuzz: OK <parses>".
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nuq_gguf.h"

static uint8_t buf[4096];
static size_t len;

static void put(const void *p, size_t n) {
    memcpy(buf + len, p, n);
    len += n;
}
static void put_u32(uint32_t v) { put(&v, 4); }
static void put_u64(uint64_t v) { put(&v, 8); }
static void put_str(const char *s) {
    put_u64(strlen(s));
    put(s, strlen(s));
}

/* gguf.zig:441-471 with the default FixtureOptions */
static void fixture(void) {
    len = 0;
    put("GGUF", 4);
    put_u32(3);
    put_u64(2);
    put_u64(3);
    put_str("general.architecture");
    put_u32(8);
    put_str("fixture");
    put_str("general.alignment");
    put_u32(4);
    put_u32(32);
    put_str("tokenizer.ggml.tokens");
    put_u32(9);
    put_u32(8);
    put_u64(2);
    put_str("a");
    put_str("unicode: \xce\xbb");
    for (int i = 0; i < 2; ++i) {
        put_str(i == 0 ? "first" : "second");
        put_u32(1);
        put_u64(4);
        put_u32(0);
        put_u64(i == 0 ? 0 : 32);
    }
    while (len % 32) buf[len++] = 0;
    memset(buf + len, 0, 64);
    len += 64;
}

static long parses = 0;

/* parse and, on success, touch everything the document exposes */
static void parse_any(const uint8_t *bytes, size_t avail, uint64_t claimed) {
    nuq_gguf *g = NULL;
    ++parses;
    if (nuq_gguf_parse(bytes, avail, claimed, NULL, &g, NULL) != NUQ_OK) {
        if (g) abort();
        return;
    }
    nuq_gguf_info info;
    if (nuq_gguf_info_get(g, &info) != NUQ_OK) abort();
    const void *dir;
    uint64_t dir_len;
    nuq_gguf_directory(g, &dir, &dir_len);
    for (uint64_t i = 0; i < info.metadata_count; ++i) {
        const char *key;
        uint64_t key_len;
        nuq_gguf_value v;
        if (nuq_gguf_metadata(g, i, &key, &key_len, &v) != NUQ_OK) abort();
        volatile char sink = key_len ? key[key_len - 1] : 0;
        (void)sink;
        if (v.kind == NUQ_GGUF_VALUE_STRING && v.string_len) sink = v.string[v.string_len - 1];
        if (v.kind == NUQ_GGUF_VALUE_ARRAY) {
            for (uint64_t k = 0; k < v.retained; ++k) {
                nuq_gguf_value item;
                if (nuq_gguf_array_value(g, i, k, &item) != NUQ_OK) abort();
            }
            nuq_gguf_array_reader r;
            if (nuq_gguf_array_reader_init(&r, v.element_type, v.count, v.file_offset, dir, dir_len, NULL) == NUQ_OK) {
                for (;;) {
                    int has = 0;
                    if (v.element_type == NUQ_GGUF_STRING) {
                        const char *s;
                        uint64_t n;
                        if (nuq_gguf_array_next_string(&r, &s, &n, &has) != NUQ_OK || !has) break;
                        if (n) sink = s[n - 1];
                    } else {
                        int32_t x;
                        if (nuq_gguf_array_next_int32(&r, &x, &has) != NUQ_OK || !has) break;
                    }
                }
            }
        }
        nuq_gguf_get(g, key, key_len, &v);
    }
    for (uint64_t i = 0; i < info.tensor_count; ++i) {
        nuq_gguf_tensor t;
        if (nuq_gguf_tensor_get(g, i, &t) != NUQ_OK) abort();
        uint64_t idx;
        if (nuq_gguf_find_tensor(g, t.name, t.name_len, &idx) != NUQ_OK) abort();
        const void *bytes_p;
        uint64_t n;
        if (nuq_gguf_tensor_bytes(g, i, &bytes_p, &n) == NUQ_OK && n) {
            volatile uint8_t sink = ((const uint8_t *)bytes_p)[n - 1];
            (void)sink;
        }
        nuq_matrix m;
        nuq_gguf_matrix(g, i, NULL, &m);
    }
    nuq_gguf_close(g);
}

int main(void) {
    fixture();
    const size_t n = len;
    uint8_t good[4096], work[4096];
    memcpy(good, buf, n);
    nuq_gguf *g = NULL;
    if (nuq_gguf_parse(good, n, n, NULL, &g, NULL) != NUQ_OK) {
        fprintf(stderr, "gguf_fuzz: the unmodified fixture was rejected\n");
        return 1;
    }
    nuq_gguf_close(g);
    for (size_t k = 0; k <= n; ++k) {
        uint8_t *copy = malloc(k ? k : 1); /* exact-size buffers: any overread is caught */
        memcpy(copy, good, k);
        parse_any(copy, k, k);
        parse_any(copy, k, n);
        parse_any(copy, k, UINT64_MAX);
        free(copy);
    }
    const uint8_t bytes8[] = {0, 1, 0x7f, 0x80, 0xff};
    const uint32_t words[] = {UINT32_MAX, 1u << 31, 13};
    const uint64_t quads[] = {UINT64_MAX, 1ull << 63, 1ull << 32, 100000, 100001};
    for (size_t at = 0; at < n; ++at) {
        for (size_t v = 0; v < sizeof bytes8; ++v) {
            memcpy(work, good, n);
            work[at] = bytes8[v];
            parse_any(work, n, n);
        }
        for (size_t v = 0; v < 3 && at + 4 <= n; ++v) {
            memcpy(work, good, n);
            memcpy(work + at, &words[v], 4);
            parse_any(work, n, n);
        }
        for (size_t v = 0; v < 5 && at + 8 <= n; ++v) {
            memcpy(work, good, n);
            memcpy(work + at, &quads[v], 8);
            parse_any(work, n, n);
        }
    }
    uint64_t state = 0x67677566ull;
    for (int round = 0; round < 200000; ++round) {
        memcpy(work, good, n);
        state = state * 6364136223846793005ull + 1442695040888963407ull;
        const int edits = 1 + (int)((state >> 33) % 4);
        for (int e = 0; e < edits; ++e) {
            state = state * 6364136223846793005ull + 1442695040888963407ull;
            work[(state >> 33) % n] = (uint8_t)(state >> 17);
        }
        parse_any(work, n, n);
    }
    printf("gguf_fuzz: OK %ld\n", parses);
    return 0;
}
