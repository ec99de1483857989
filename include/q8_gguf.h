/* q8_gguf.h: a GGUF v3 model file's header and tensor table, and the upload of its Q8_0 tensors
 * to HBM for the products of q8_rt.h.
 *
 * The reader replaces the reference's header reader (src/host/gguf_reader.h:1-60): the same structs
 * and results (fields, key text, offsets, sizes), under rt_gguf_ names so that both can be linked
 * into one program; its own error texts. The upload follows the reference engine's load
 * loop (src/card/engine.c:287-316): every Q8_0 tensor once per distinct file offset, so tensors
 * tied by offset share one handle (engine.c:307-310).
 *
 * Only pointers and integers cross this interface; a failed call returns -1 with "path: reason"
 * in err (never aborts on a bad file). One host thread, as the rest of q8_rt.h. */
#ifndef Q8_GGUF_H
#define Q8_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "q8_rt.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF metadata value types (gguf_reader.h:12) */
enum { RT_GGUF_U8, RT_GGUF_I8, RT_GGUF_U16, RT_GGUF_I16, RT_GGUF_U32, RT_GGUF_I32, RT_GGUF_F32, RT_GGUF_BOOL, RT_GGUF_STR, RT_GGUF_ARR,
       RT_GGUF_U64, RT_GGUF_I64, RT_GGUF_F64 };
/* the ggml tensor types the products take (gguf_reader.h:15) */
enum { RT_GGML_F32 = 0, RT_GGML_Q8_0 = 8 };
/* one past the largest ggml type id the reader knows (gguf_reader.h:58) */
#define RT_GGUF_MAX_TENSOR_TYPE 43

/* A metadata key (gguf_reader.h:17-23). */
struct rt_gguf_key {
    char name[96];
    uint32_t type;      /* RT_GGUF_* */
    uint32_t elem_type; /* for RT_GGUF_ARR */
    uint64_t n;         /* an array's count; a string's length in the file (text may hold less) */
    char text[128];     /* printable value: integers in decimal, f32 to 9 and f64 to 17 significant
                           digits, bool true/false, a string's first 127 bytes; an array of at most
                           16 numbers as its values with one space between, any other array "" */
};

/* A tensor of the table (gguf_reader.h:25-32), and its HBM handle once uploaded. */
struct rt_gguf_tensor {
    char name[96];
    uint32_t n_dims;
    uint64_t dim[4];  /* ne0 first: the contiguous dimension (cols of a matrix) */
    uint32_t type;    /* ggml type id */
    uint64_t offset;  /* absolute offset in the file */
    uint64_t bytes;
    const void *w;    /* after rt_gguf_upload: a Q8_0 matrix's handle (rows = dim[1]*dim[2]*dim[3],
                         cols = dim[0]), shared by every tensor at the same offset; else NULL */
};

/* A file's header (gguf_reader.h:34-43). */
struct rt_gguf {
    uint32_t version;
    uint64_t file_size;
    uint64_t header_end, data_start;
    uint64_t data_bytes; /* bytes of all tensors together, ties counted each time */
    uint64_t need;       /* data_start + the end of the furthest tensor: the least size a whole file has */
    uint64_t n_keys, n_tensors;
    struct rt_gguf_key *keys;
    struct rt_gguf_tensor *tensors;
    uint64_t q8_bytes;   /* after rt_gguf_upload: HBM bytes of the distinct Q8_0 matrices */
    int q8_count;        /* and their number */
};

/* Reads the header of path into g (in place of gguf_load, gguf_reader.c:166-218). 0, or -1 with
 * "path: reason" in err, the reason naming the byte where the header went wrong: the file cannot be
 * opened, does not start with "GGUF", ends inside the header, declares more keys or tensors than
 * its size could hold, uses a value type GGUF does not define, has a tensor of more than 4
 * dimensions or of an unknown ggml type, or an alignment of 0. general.alignment is read as the
 * reference reads it, strtoull of the key's text whatever its type (32 when absent). Refused here
 * where the reference's arithmetic would wrap 64 bits: a tensor whose offset + size overflows, an
 * alignment or a data end that puts the data past 2^64 bytes. The file is mapped, never read past
 * the header. */
int rt_gguf_read(struct rt_gguf *g, const char *path, char *err, size_t err_cap);
/* Frees the tables (gguf_free). Handles are not freed here: rt_gguf_release does that. */
void rt_gguf_free(struct rt_gguf *g);

/* Lookups by name (gguf_reader.c:228-242); NULL if absent. */
const struct rt_gguf_key *rt_gguf_key(const struct rt_gguf *g, const char *name);
const struct rt_gguf_tensor *rt_gguf_tensor(const struct rt_gguf *g, const char *name);
/* The tensor at an absolute file offset, as the reference engine binds its slots (engine.c:307-310). */
const struct rt_gguf_tensor *rt_gguf_tensor_at(const struct rt_gguf *g, uint64_t offset);
/* A scalar key's value as an unsigned integer, or fallback if absent (gguf_reader.c:244-248). */
uint64_t rt_gguf_key_u64(const struct rt_gguf *g, const char *name, uint64_t fallback);
/* Names: "u8".."f64" ("?" past them), and a ggml type's name or NULL for an unknown id
 * (gguf_reader.c:33-42). */
const char *rt_gguf_value_type_name(uint32_t type);
const char *rt_gguf_tensor_type_name(uint32_t type);

/* Uploads every Q8_0 tensor of the file g was read from to HBM in form S (rt_q8_upload_fd), once
 * per distinct offset, and sets tensors[i].w. -1 with the reason in err, and nothing left
 * uploaded, when the file is shorter than its tensor table needs, a Q8_0 tensor is not a matrix the
 * products take (rows = dim[1]*dim[2]*dim[3] a multiple of 16, cols = dim[0] of 32), a read fails,
 * or HBM is full. Other types stay in the file (their offset and bytes are in the table). */
int rt_gguf_upload(struct rt *R, struct rt_gguf *g, const char *path, char *err, size_t err_cap);
/* Frees the handles rt_gguf_upload made (each distinct one once) and clears tensors[i].w. */
void rt_gguf_release(struct rt *R, struct rt_gguf *g);

#ifdef __cplusplus
}
#endif

#endif
