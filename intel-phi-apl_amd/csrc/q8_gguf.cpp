/* q8_gguf.cpp: the GGUF v3 header reader and the Q8_0 upload of include/q8_gguf.h.
 *
 * GGUF v3, little endian: "GGUF", u32 version, u64 tensor count, u64 key count; the keys (a string
 * name, u32 value type, the value; a string is u64 length + bytes; an array is u32 element type, u64
 * count, the elements); the tensor table (name, u32 dimension count, u64 dimensions ne0 first, u32
 * ggml type, u64 offset from the data start); then the data, from the first multiple of
 * general.alignment (32 when absent) at or after the table's end.
 *
 * The file is mapped read-only and the header parsed in place by a cursor that checks every read
 * against the bytes left (a count that the rest of the file cannot hold is refused before anything
 * is allocated for it). Values are decoded to a typed scalar and formatted into the key's text
 * afterwards. Only the header is touched; the upload reads each Q8_0 tensor's bytes with pread.
 * Results (fields, key text, offsets, sizes) are held field for field to the reference's reader
 * (src/host/gguf_reader.c) on synthetic files in the tests; the error texts are this file's own,
 * with the byte offset where the header went wrong. An alignment of 0 is refused. */
#include "../../include/q8_gguf.h"

#include <errno.h>
#include <fcntl.h>
#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <unordered_map>

namespace {

/* ggml's types: name, elements a block, bytes a block (llama.cpp f5b9bd3 ggml/src/ggml.c
 * type_traits). Ids without a type (4, 5, 31-33, 36-38) have no name. */
struct ggml_type {
    const char *name;
    uint32_t block, bytes;
};

ggml_type ggml_type_of(uint32_t id)
{
    switch (id) {
    case 0: return {"F32", 1, 4};
    case 1: return {"F16", 1, 2};
    case 2: return {"Q4_0", 32, 18};
    case 3: return {"Q4_1", 32, 20};
    case 6: return {"Q5_0", 32, 22};
    case 7: return {"Q5_1", 32, 24};
    case 8: return {"Q8_0", 32, 34};
    case 9: return {"Q8_1", 32, 36};
    case 10: return {"Q2_K", 256, 84};
    case 11: return {"Q3_K", 256, 110};
    case 12: return {"Q4_K", 256, 144};
    case 13: return {"Q5_K", 256, 176};
    case 14: return {"Q6_K", 256, 210};
    case 15: return {"Q8_K", 256, 292};
    case 16: return {"IQ2_XXS", 256, 66};
    case 17: return {"IQ2_XS", 256, 74};
    case 18: return {"IQ3_XXS", 256, 98};
    case 19: return {"IQ1_S", 256, 50};
    case 20: return {"IQ4_NL", 32, 18};
    case 21: return {"IQ3_S", 256, 110};
    case 22: return {"IQ2_S", 256, 82};
    case 23: return {"IQ4_XS", 256, 136};
    case 24: return {"I8", 1, 1};
    case 25: return {"I16", 1, 2};
    case 26: return {"I32", 1, 4};
    case 27: return {"I64", 1, 8};
    case 28: return {"F64", 1, 8};
    case 29: return {"IQ1_M", 256, 56};
    case 30: return {"BF16", 1, 2};
    case 34: return {"TQ1_0", 256, 54};
    case 35: return {"TQ2_0", 256, 66};
    case 39: return {"MXFP4", 32, 17};
    case 40: return {"NVFP4", 64, 36};
    case 41: return {"Q1_0", 128, 18};
    case 42: return {"Q2_0", 64, 18};
    default: return {nullptr, 0, 0};
    }
}

/* width in bytes of a scalar GGUF value type; 0 for string, array and unknown ids */
unsigned width_of(uint32_t t)
{
    static const unsigned w[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    return t < sizeof w / sizeof w[0] ? w[t] : 0;
}

/* a decoded scalar: its type and its bits, widened */
struct scalar {
    uint32_t type;
    uint64_t bits;
};

/* the value's text: decimal integers, f32 with 9 and f64 with 17 significant digits (each exact on
 * a round trip), bool as true/false */
void format(const scalar &v, char *out, size_t cap)
{
    switch (v.type) {
    case RT_GGUF_U8: case RT_GGUF_U16: case RT_GGUF_U32: case RT_GGUF_U64:
        snprintf(out, cap, "%" PRIu64, v.bits);
        break;
    case RT_GGUF_I8: snprintf(out, cap, "%d", (int)(int8_t)v.bits); break;
    case RT_GGUF_I16: snprintf(out, cap, "%d", (int)(int16_t)v.bits); break;
    case RT_GGUF_I32: snprintf(out, cap, "%" PRId32, (int32_t)v.bits); break;
    case RT_GGUF_I64: snprintf(out, cap, "%" PRId64, (int64_t)v.bits); break;
    case RT_GGUF_BOOL: snprintf(out, cap, "%s", v.bits ? "true" : "false"); break;
    case RT_GGUF_F32: {
        float f;
        const uint32_t b = (uint32_t)v.bits;
        memcpy(&f, &b, 4);
        snprintf(out, cap, "%.9g", (double)f);
        break;
    }
    default: {
        double d;
        memcpy(&d, &v.bits, 8);
        snprintf(out, cap, "%.17g", d);
        break;
    }
    }
}

/* A cursor over the mapped header. Every read checks the bytes left; the first failure is kept
 * (what, and the offset where it happened) and every later read fails at once. */
class cursor {
  public:
    cursor(const uint8_t *base, uint64_t size) : base_(base), at_(0), size_(size) {}

    bool ok() const { return !what_; }
    uint64_t offset() const { return at_; }
    const char *what() const { return what_; }
    uint64_t where() const { return where_; }
    uint64_t left() const { return size_ - at_; }

    bool fail(const char *what)
    {
        if (!what_) {
            what_ = what;
            where_ = at_;
        }
        return false;
    }
    /* n bytes at the cursor, or NULL (failed: the header ends inside them) */
    const uint8_t *take(uint64_t n)
    {
        if (what_)
            return nullptr;
        if (n > left()) {
            fail("the header ends inside a field");
            return nullptr;
        }
        const uint8_t *p = base_ + at_;
        at_ += n;
        return p;
    }
    template <class T>
    T le()
    {
        T v = 0;
        if (const uint8_t *p = take(sizeof(T)))
            memcpy(&v, p, sizeof(T)); /* GGUF is little endian, as this host */
        return v;
    }
    /* a string: its first cap-1 bytes into buf (NUL-terminated), the full length returned */
    uint64_t text(char *buf, size_t cap)
    {
        const uint64_t n = le<uint64_t>();
        const uint8_t *p = take(n);
        const size_t keep = p ? (size_t)(n < cap - 1 ? n : cap - 1) : 0;
        if (keep)
            memcpy(buf, p, keep);
        buf[keep] = 0;
        return n;
    }
    /* one scalar of type t */
    bool value(uint32_t t, scalar *v)
    {
        const unsigned w = width_of(t);
        if (!w)
            return fail("a key has a value type GGUF does not define");
        const uint8_t *p = take(w);
        if (!p)
            return false;
        v->type = t;
        v->bits = 0;
        memcpy(&v->bits, p, w);
        return true;
    }

  private:
    const uint8_t *base_;
    uint64_t at_, size_;
    const char *what_ = nullptr;
    uint64_t where_ = 0;
};

/* one metadata key into k; its unsigned value in *num when it is an integer scalar */
bool parse_key(cursor &c, struct rt_gguf_key &k, bool *integer, uint64_t *num)
{
    c.text(k.name, sizeof k.name);
    k.type = c.le<uint32_t>();
    k.elem_type = 0;
    k.n = 1;
    k.text[0] = 0;
    *integer = false;
    if (!c.ok())
        return false;
    if (k.type == RT_GGUF_STR) {
        k.n = c.text(k.text, sizeof k.text);
        return c.ok();
    }
    if (k.type != RT_GGUF_ARR) {
        scalar v;
        if (!c.value(k.type, &v))
            return false;
        format(v, k.text, sizeof k.text);
        *integer = k.type != RT_GGUF_F32 && k.type != RT_GGUF_F64 && k.type != RT_GGUF_BOOL;
        *num = v.bits;
        return true;
    }
    k.elem_type = c.le<uint32_t>();
    k.n = c.le<uint64_t>();
    if (!c.ok())
        return false;
    if (k.elem_type == RT_GGUF_STR) { /* strings: stepped over, no text */
        for (uint64_t j = 0; j < k.n && c.ok(); j++) {
            const uint64_t len = c.le<uint64_t>();
            c.take(len);
        }
        return c.ok();
    }
    const unsigned w = width_of(k.elem_type);
    if (!w)
        return c.fail("an array has an element type GGUF does not define");
    if (k.n > c.left() / w)
        return c.fail("the header ends inside an array");
    if (k.n > 16) { /* long numeric arrays: stepped over, no text */
        c.take(k.n * w);
        return c.ok();
    }
    size_t at = 0;
    for (uint64_t j = 0; j < k.n; j++) {
        scalar v;
        if (!c.value(k.elem_type, &v))
            return false;
        char one[40];
        format(v, one, sizeof one);
        at += (size_t)snprintf(k.text + at, at < sizeof k.text ? sizeof k.text - at : 0, j ? " %s" : "%s", one);
        if (at >= sizeof k.text)
            at = sizeof k.text - 1;
    }
    return true;
}

/* one entry of the tensor table into t (offset still relative to the data start) */
bool parse_tensor(cursor &c, struct rt_gguf_tensor &t)
{
    c.text(t.name, sizeof t.name);
    t.n_dims = c.le<uint32_t>();
    if (!c.ok())
        return false;
    if (t.n_dims > 4)
        return c.fail("a tensor has more than 4 dimensions");
    uint64_t elements = 1; /* wraps on absurd dimensions: the upload checks those */
    for (uint32_t d = 0; d < 4; d++) {
        t.dim[d] = d < t.n_dims ? c.le<uint64_t>() : 0;
        if (d < t.n_dims)
            elements *= t.dim[d];
    }
    t.type = c.le<uint32_t>();
    t.offset = c.le<uint64_t>();
    if (!c.ok())
        return false;
    const ggml_type g = ggml_type_of(t.type);
    if (!g.name)
        return c.fail("a tensor has a ggml type id this reader does not know");
    t.bytes = elements / g.block * g.bytes;
    t.w = nullptr;
    return true;
}

void message(char *err, size_t cap, const char *path, const char *why)
{
    if (err && cap)
        snprintf(err, cap, "%s: %s", path, why);
}

/* the header of the mapped file into g; false with the reason in why */
bool parse(struct rt_gguf *g, const uint8_t *base, uint64_t size, char *why, size_t why_cap)
{
    cursor c(base, size);
    const uint8_t *magic = c.take(4);
    if (magic && memcmp(magic, "GGUF", 4) != 0) {
        snprintf(why, why_cap, "not a GGUF file: it starts with %02x %02x %02x %02x, not \"GGUF\"", magic[0], magic[1], magic[2], magic[3]);
        return false;
    }
    g->version = c.le<uint32_t>();
    g->n_tensors = c.le<uint64_t>();
    g->n_keys = c.le<uint64_t>();
    /* a key takes at least 12 bytes (empty name, type, a u8), a tensor at least 24 */
    if (c.ok() && (g->n_keys > c.left() / 12 || g->n_tensors > c.left() / 24))
        c.fail("the header ends before its keys and tensors (counts larger than the file holds)");
    if (c.ok()) {
        g->keys = (struct rt_gguf_key *)calloc(g->n_keys ? g->n_keys : 1, sizeof *g->keys);
        g->tensors = (struct rt_gguf_tensor *)calloc(g->n_tensors ? g->n_tensors : 1, sizeof *g->tensors);
        if (!g->keys || !g->tensors) {
            snprintf(why, why_cap, "out of memory for %" PRIu64 " keys and %" PRIu64 " tensors", g->n_keys, g->n_tensors);
            return false;
        }
    }
    /* general.alignment as the reference reads it: strtoull of the key's text, whatever its type
     * (gguf_reader.c:198-202), so a string "64" or an f32 64 give 64 */
    uint64_t alignment = 32;
    for (uint64_t i = 0; i < g->n_keys && c.ok(); i++) {
        bool integer = false;
        uint64_t num = 0;
        if (parse_key(c, g->keys[i], &integer, &num) && strcmp(g->keys[i].name, "general.alignment") == 0)
            alignment = strtoull(g->keys[i].text, nullptr, 10);
    }
    uint64_t data_end = 0;
    for (uint64_t i = 0; i < g->n_tensors && c.ok(); i++) {
        struct rt_gguf_tensor &t = g->tensors[i];
        if (!parse_tensor(c, t))
            break;
        /* an offset and size whose end wraps 64 bits would pass every later size check */
        if (t.bytes > UINT64_MAX - t.offset) {
            snprintf(why, why_cap, "tensor %s: offset %" PRIu64 " + %" PRIu64 " bytes overflows 64 bits", t.name, t.offset, t.bytes);
            return false;
        }
        g->data_bytes += t.bytes;
        data_end = t.offset + t.bytes > data_end ? t.offset + t.bytes : data_end;
    }
    if (!c.ok()) {
        snprintf(why, why_cap, "%s (at byte %" PRIu64 " of %" PRIu64 ")", c.what(), c.where(), size);
        return false;
    }
    if (alignment == 0) {
        snprintf(why, why_cap, "general.alignment is 0");
        return false;
    }
    g->header_end = c.offset();
    /* the reference's arithmetic wraps for an alignment near 2^64 (a negative key, for example);
     * such a file is refused here */
    if (alignment - 1 > UINT64_MAX - g->header_end) {
        snprintf(why, why_cap, "general.alignment %" PRIu64 " puts the data past 2^64 bytes", alignment);
        return false;
    }
    g->data_start = (g->header_end + alignment - 1) / alignment * alignment;
    if (data_end > UINT64_MAX - g->data_start) {
        snprintf(why, why_cap, "the tensors end past 2^64 bytes (data at %" PRIu64 ", their end %" PRIu64 " past it)", g->data_start, data_end);
        return false;
    }
    g->need = g->data_start + data_end;
    for (uint64_t i = 0; i < g->n_tensors; i++)
        g->tensors[i].offset += g->data_start;
    return true;
}

} // namespace

extern "C" {

int rt_gguf_read(struct rt_gguf *g, const char *path, char *err, size_t err_cap)
{
    memset(g, 0, sizeof *g);
    const int fd = open(path, O_RDONLY);
    struct stat st;
    if (fd < 0 || fstat(fd, &st) != 0) {
        message(err, err_cap, path, strerror(errno));
        if (fd >= 0)
            close(fd);
        return -1;
    }
    if (!S_ISREG(st.st_mode)) {
        message(err, err_cap, path, S_ISDIR(st.st_mode) ? strerror(EISDIR) : "not a regular file");
        close(fd);
        return -1;
    }
    g->file_size = (uint64_t)st.st_size;
    char why[256] = "the header ends inside a field (at byte 0 of 0)";
    bool ok = false;
    if (st.st_size > 0) {
        void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            snprintf(why, sizeof why, "%s", strerror(errno));
        } else {
            ok = parse(g, (const uint8_t *)m, (uint64_t)st.st_size, why, sizeof why);
            munmap(m, (size_t)st.st_size);
        }
    }
    close(fd);
    if (!ok) {
        const uint64_t size = g->file_size;
        rt_gguf_free(g);
        memset(g, 0, sizeof *g);
        g->file_size = size;
        message(err, err_cap, path, why);
        return -1;
    }
    return 0;
}

void rt_gguf_free(struct rt_gguf *g)
{
    free(g->keys);
    free(g->tensors);
    g->keys = nullptr;
    g->tensors = nullptr;
}

const struct rt_gguf_key *rt_gguf_key(const struct rt_gguf *g, const char *name)
{
    for (uint64_t i = 0; i < g->n_keys; i++)
        if (strcmp(g->keys[i].name, name) == 0)
            return &g->keys[i];
    return nullptr;
}

const struct rt_gguf_tensor *rt_gguf_tensor(const struct rt_gguf *g, const char *name)
{
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (strcmp(g->tensors[i].name, name) == 0)
            return &g->tensors[i];
    return nullptr;
}

const struct rt_gguf_tensor *rt_gguf_tensor_at(const struct rt_gguf *g, uint64_t offset)
{
    for (uint64_t i = 0; i < g->n_tensors; i++)
        if (g->tensors[i].offset == offset)
            return &g->tensors[i];
    return nullptr;
}

uint64_t rt_gguf_key_u64(const struct rt_gguf *g, const char *name, uint64_t fallback)
{
    const struct rt_gguf_key *k = rt_gguf_key(g, name);
    return k ? strtoull(k->text, nullptr, 10) : fallback;
}

const char *rt_gguf_value_type_name(uint32_t type)
{
    static const char *const names[] = {"u8", "i8", "u16", "i16", "u32", "i32", "f32", "bool", "str", "arr", "u64", "i64", "f64"};
    return type < sizeof names / sizeof names[0] ? names[type] : "?";
}

const char *rt_gguf_tensor_type_name(uint32_t type)
{
    return ggml_type_of(type).name;
}

void rt_gguf_release(struct rt *R, struct rt_gguf *g)
{
    std::unordered_map<const void *, bool> freed;
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const void *w = g->tensors[i].w;
        if (w && !freed[w]) {
            rt_q8_free(R, w);
            freed[w] = true;
        }
        g->tensors[i].w = nullptr;
    }
    g->q8_bytes = 0;
    g->q8_count = 0;
}

int rt_gguf_upload(struct rt *R, struct rt_gguf *g, const char *path, char *err, size_t err_cap)
{
    char why[256];
    if (g->file_size < g->need) {
        snprintf(why, sizeof why, "truncated: the file is %" PRIu64 " B short of its tensor table", g->need - g->file_size);
        message(err, err_cap, path, why);
        return -1;
    }
    const int fd = open(path, O_RDONLY);
    struct stat st;
    if (fd < 0 || fstat(fd, &st) != 0 || (uint64_t)st.st_size < g->need) {
        message(err, err_cap, path, fd < 0 ? strerror(errno) : "the file is shorter than its tensor table");
        if (fd >= 0)
            close(fd);
        return -1;
    }
    std::unordered_map<uint64_t, uint64_t> first; /* offset -> the first tensor there */
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        struct rt_gguf_tensor &t = g->tensors[i];
        if (t.type != RT_GGML_Q8_0)
            continue;
        /* rows = dim[1]*dim[2]*dim[3], bounded (2^32 rows, 2^28 columns) before anything is
         * multiplied, so that no size below overflows and the upload gets sane longs */
        uint64_t rows = 1;
        bool sane = t.dim[0] <= (1ull << 28);
        for (uint32_t d = 1; d < t.n_dims && sane; d++) {
            sane = t.dim[d] <= (1ull << 32) && rows * t.dim[d] <= (1ull << 32);
            rows *= t.dim[d];
        }
        const uint64_t cols = t.n_dims ? t.dim[0] : 0;
        if (!sane) {
            snprintf(why, sizeof why, "tensor %s: its dimensions are out of range", t.name);
            goto fail;
        }
        if (t.n_dims < 2 || rows == 0 || rows % 16 || cols == 0 || cols % 32 || rows * cols / 32 * 34 != t.bytes) {
            snprintf(why, sizeof why, "tensor %s: %" PRIu64 " rows x %" PRIu64 " columns is not a matrix the products take (rows a multiple of 16, columns of 32)",
                     t.name, rows, cols);
            goto fail;
        }
        {
            auto seen = first.find(t.offset);
            if (seen != first.end()) {
                const struct rt_gguf_tensor &s = g->tensors[seen->second];
                if (s.dim[0] != t.dim[0] || s.bytes != t.bytes) {
                    snprintf(why, sizeof why, "tensors %s and %s share an offset with different shapes", s.name, t.name);
                    goto fail;
                }
                t.w = s.w; /* tied: one matrix, one handle (engine.c:307-310) */
                continue;
            }
            errno = 0;
            t.w = rt_q8_upload_fd(R, fd, t.offset, (long)rows, (long)cols);
            if (!t.w) {
                snprintf(why, sizeof why, "tensor %s: %s", t.name, errno == ENOMEM ? "HBM is full" : strerror(errno ? errno : EIO));
                goto fail;
            }
            first[t.offset] = i;
            g->q8_bytes += t.bytes;
            g->q8_count++;
        }
    }
    close(fd);
    return 0;
fail:
    close(fd);
    rt_gguf_release(R, g);
    message(err, err_cap, path, why);
    return -1;
}

} /* extern "C" */
