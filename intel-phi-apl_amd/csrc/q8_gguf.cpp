/* q8_gguf.cpp: the GGUF v3 header reader and the Q8_0 upload of include/q8_gguf.h.
 *
 * A GGUF v3 file is: "GGUF", u32 version, u64 tensor count, u64 key count; the keys (u64-length
 * string name, u32 value type, the value; an array is u32 element type, u64 count, the elements);
 * the tensor table (name, u32 dimension count, u64 dimensions ne0 first, u32 ggml type, u64 offset
 * from the data start); then, at the next multiple of general.alignment (32 by default), the data.
 * Only the header is read here; the upload reads each Q8_0 tensor's bytes with pread.
 *
 * The reader's results (fields, value text, errors) are the reference's (src/host/gguf_reader.c:
 * 87-218), checked on synthetic files against it built from its source. One difference: an
 * alignment of 0, on which the reference divides by zero, is an error here. */
#include "../../include/q8_gguf.h"

#include <errno.h>
#include <fcntl.h>
#include <inttypes.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#include <unordered_map>

namespace {

/* ggml's types: name, elements a block, bytes a block (llama.cpp f5b9bd3 ggml/src/ggml.c
 * type_traits; gguf_reader.c:18-30). Ids without a type (4, 5, 31-33, 36-38) give a null name. */
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

/* Bytes of a scalar value type; 0 for a string, an array or an unknown type. */
size_t scalar_bytes(uint32_t t)
{
    switch (t) {
    case RT_GGUF_U8: case RT_GGUF_I8: case RT_GGUF_BOOL: return 1;
    case RT_GGUF_U16: case RT_GGUF_I16: return 2;
    case RT_GGUF_U32: case RT_GGUF_I32: case RT_GGUF_F32: return 4;
    case RT_GGUF_U64: case RT_GGUF_I64: case RT_GGUF_F64: return 8;
    default: return 0;
    }
}

/* Thrown by the reader; rt_gguf_read turns it into "path: reason". */
struct bad_file {
    const char *why;
};

/* Sequential reads of the header from a stdio stream. */
class header {
  public:
    explicit header(FILE *f) : f_(f) {}

    [[noreturn]] static void fail(const char *why) { throw bad_file{why}; }

    void read(void *p, size_t n)
    {
        if (fread(p, 1, n, f_) != n)
            fail(feof(f_) ? "unexpected end of file in the header" : strerror(errno));
    }
    uint32_t u32()
    {
        uint32_t v;
        read(&v, 4);
        return v;
    }
    uint64_t u64()
    {
        uint64_t v;
        read(&v, 8);
        return v;
    }
    void skip(uint64_t n, const char *why)
    {
        if (fseeko(f_, (off_t)n, SEEK_CUR) != 0)
            fail(why);
    }
    /* A string (u64 length, bytes): the first cap-1 bytes into buf, the rest skipped; returns the
     * full length. */
    uint64_t string(char *buf, size_t cap)
    {
        const uint64_t n = u64();
        const size_t keep = n < cap - 1 ? (size_t)n : cap - 1;
        read(buf, keep);
        buf[keep] = 0;
        if (n > keep)
            skip(n - keep, "seek in a string");
        return n;
    }
    /* One scalar of type t, as text. */
    void scalar(uint32_t t, char *out, size_t cap)
    {
        const size_t n = scalar_bytes(t);
        if (!n)
            fail("bad value type");
        unsigned char b[8];
        read(b, n);
        union {
            uint8_t u8;
            int8_t i8;
            uint16_t u16;
            int16_t i16;
            uint32_t u32;
            int32_t i32;
            float f32;
            uint64_t u64;
            int64_t i64;
            double f64;
        } v;
        memcpy(&v, b, n);
        switch (t) {
        case RT_GGUF_U8: snprintf(out, cap, "%u", (unsigned)v.u8); break;
        case RT_GGUF_I8: snprintf(out, cap, "%d", (int)v.i8); break;
        case RT_GGUF_BOOL: snprintf(out, cap, "%s", v.u8 ? "true" : "false"); break;
        case RT_GGUF_U16: snprintf(out, cap, "%u", (unsigned)v.u16); break;
        case RT_GGUF_I16: snprintf(out, cap, "%d", (int)v.i16); break;
        case RT_GGUF_U32: snprintf(out, cap, "%" PRIu32, v.u32); break;
        case RT_GGUF_I32: snprintf(out, cap, "%" PRId32, v.i32); break;
        case RT_GGUF_F32: snprintf(out, cap, "%.9g", (double)v.f32); break;
        case RT_GGUF_U64: snprintf(out, cap, "%" PRIu64, v.u64); break;
        case RT_GGUF_I64: snprintf(out, cap, "%" PRId64, v.i64); break;
        default: snprintf(out, cap, "%.17g", v.f64); break;
        }
    }
    void key(struct rt_gguf_key &k)
    {
        string(k.name, sizeof k.name);
        k.type = u32();
        k.elem_type = 0;
        k.n = 1;
        k.text[0] = 0;
        if (k.type == RT_GGUF_STR) {
            k.n = string(k.text, sizeof k.text);
        } else if (k.type == RT_GGUF_ARR) {
            k.elem_type = u32();
            k.n = u64();
            if (k.elem_type == RT_GGUF_STR) {
                char none[8];
                for (uint64_t j = 0; j < k.n; j++)
                    string(none, sizeof none);
            } else if (k.n <= 16) {
                for (uint64_t j = 0; j < k.n; j++) {
                    char one[32];
                    scalar(k.elem_type, one, sizeof one);
                    const size_t at = strlen(k.text);
                    snprintf(k.text + at, sizeof k.text - at, "%s%s", j ? " " : "", one);
                }
            } else {
                const size_t each = scalar_bytes(k.elem_type);
                if (!each)
                    fail("bad value type");
                skip(k.n * each, "seek over an array");
            }
        } else {
            scalar(k.type, k.text, sizeof k.text);
        }
    }
    void tensor(struct rt_gguf_tensor &t)
    {
        string(t.name, sizeof t.name);
        t.n_dims = u32();
        if (t.n_dims > 4)
            fail("tensor with more than 4 dimensions");
        uint64_t elements = 1;
        for (uint32_t d = 0; d < t.n_dims; d++)
            elements *= (t.dim[d] = u64());
        t.type = u32();
        t.offset = u64(); /* from the data start; made absolute once it is known */
        const ggml_type g = ggml_type_of(t.type);
        if (!g.name)
            fail("tensor of an unknown ggml type");
        t.bytes = elements / g.block * g.bytes;
        t.w = nullptr;
    }
    off_t tell() const { return ftello(f_); }

  private:
    FILE *f_;
};

void message(char *err, size_t cap, const char *path, const char *why)
{
    if (err && cap)
        snprintf(err, cap, "%s: %s", path, why);
}

} // namespace

extern "C" {

int rt_gguf_read(struct rt_gguf *g, const char *path, char *err, size_t err_cap)
{
    memset(g, 0, sizeof *g);
    FILE *f = fopen(path, "rb");
    struct stat st;
    if (!f || fstat(fileno(f), &st) != 0) {
        message(err, err_cap, path, strerror(errno));
        if (f)
            fclose(f);
        return -1;
    }
    try {
        header h(f);
        char magic[4];
        h.read(magic, 4);
        if (memcmp(magic, "GGUF", 4) != 0)
            header::fail("not a GGUF file (magic)");
        g->version = h.u32();
        g->n_tensors = h.u64();
        g->n_keys = h.u64();
        g->file_size = (uint64_t)st.st_size;
        g->keys = (struct rt_gguf_key *)calloc(g->n_keys ? g->n_keys : 1, sizeof *g->keys);
        g->tensors = (struct rt_gguf_tensor *)calloc(g->n_tensors ? g->n_tensors : 1, sizeof *g->tensors);
        if (!g->keys || !g->tensors)
            header::fail("out of memory");
        uint64_t alignment = 32, data_end = 0;
        for (uint64_t i = 0; i < g->n_keys; i++) {
            h.key(g->keys[i]);
            if (strcmp(g->keys[i].name, "general.alignment") == 0)
                alignment = strtoull(g->keys[i].text, nullptr, 10);
        }
        for (uint64_t i = 0; i < g->n_tensors; i++) {
            struct rt_gguf_tensor &t = g->tensors[i];
            h.tensor(t);
            g->data_bytes += t.bytes;
            if (t.offset + t.bytes > data_end)
                data_end = t.offset + t.bytes;
        }
        if (alignment == 0)
            header::fail("general.alignment is 0");
        g->header_end = (uint64_t)h.tell();
        g->data_start = (g->header_end + alignment - 1) / alignment * alignment;
        g->need = g->data_start + data_end;
        for (uint64_t i = 0; i < g->n_tensors; i++)
            g->tensors[i].offset += g->data_start;
    } catch (const bad_file &e) {
        message(err, err_cap, path, e.why);
        fclose(f);
        rt_gguf_free(g);
        return -1;
    }
    fclose(f);
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
