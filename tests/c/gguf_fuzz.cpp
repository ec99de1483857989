/* gguf_fuzz.cpp: the GGUF header reader (intel-phi-apl_amd/csrc/q8_gguf.cpp) on a list of files, for
 * tests/test_gguf_fuzz.py, which builds it with AddressSanitizer and UndefinedBehaviorSanitizer and
 * feeds it seeded corruptions of valid files. Each file is read; a refused one must say why in
 * "path: reason" form, and an accepted one must hold the header's invariants (printed as
 * "VIOLATION ..." lines otherwise): the header inside the file, the data after the header, every
 * tensor at most 4-D, of a known type, inside [data_start, need) without 64-bit wrap, every name and
 * text terminated, every tensor found again by its name and by its offset. The harness never
 * uploads, so the two upload calls the reader's object refers to abort if reached.
 * Usage: gguf_fuzz LISTFILE (one path a line); prints "accepted A refused R". */
#include "q8_gguf.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

extern "C" const void *rt_q8_upload_fd(struct rt *, int, uint64_t, long, long)
{
    abort();
}

extern "C" void rt_q8_free(struct rt *, const void *)
{
    abort();
}

static long violations = 0;

static void violation(const char *path, const char *what, unsigned long long a, unsigned long long b)
{
    printf("VIOLATION %s: %s (%llu, %llu)\n", path, what, a, b);
    violations++;
}

static void check(const char *path, const struct rt_gguf *g)
{
    if (g->header_end > g->file_size)
        violation(path, "header ends past the file", g->header_end, g->file_size);
    if (g->data_start < g->header_end)
        violation(path, "data starts inside the header", g->data_start, g->header_end);
    for (uint64_t i = 0; i < g->n_keys; i++) {
        const struct rt_gguf_key *k = &g->keys[i];
        if (!memchr(k->name, 0, sizeof k->name) || !memchr(k->text, 0, sizeof k->text))
            violation(path, "a key's name or text is not terminated", i, 0);
        else if (rt_gguf_key(g, k->name) == NULL)
            violation(path, "a key is not found by its name", i, 0);
    }
    for (uint64_t i = 0; i < g->n_tensors; i++) {
        const struct rt_gguf_tensor *t = &g->tensors[i];
        if (!memchr(t->name, 0, sizeof t->name)) {
            violation(path, "a tensor's name is not terminated", i, 0);
            continue;
        }
        if (t->n_dims > 4)
            violation(path, "a tensor of more than 4 dimensions", i, t->n_dims);
        if (t->type >= RT_GGUF_MAX_TENSOR_TYPE)
            violation(path, "a tensor of an unknown type", i, t->type);
        if (t->offset < g->data_start)
            violation(path, "a tensor before the data", t->offset, g->data_start);
        if (t->offset + t->bytes < t->offset)
            violation(path, "a tensor's end wraps 64 bits", t->offset, t->bytes);
        else if (t->offset + t->bytes > g->need)
            violation(path, "a tensor ends past `need`", t->offset + t->bytes, g->need);
        if (rt_gguf_tensor(g, t->name) == NULL)
            violation(path, "a tensor is not found by its name", i, 0);
        const struct rt_gguf_tensor *at = rt_gguf_tensor_at(g, t->offset);
        if (at == NULL || at->offset != t->offset)
            violation(path, "a tensor is not found by its offset", i, t->offset);
    }
    (void)rt_gguf_key_u64(g, "general.alignment", 32);
}

int main(int argc, char **argv)
{
    if (argc != 2) {
        fprintf(stderr, "usage: gguf_fuzz LISTFILE\n");
        return 2;
    }
    FILE *list = fopen(argv[1], "r");
    if (!list) {
        perror(argv[1]);
        return 2;
    }
    char path[4096];
    long accepted = 0, refused = 0;
    while (fgets(path, sizeof path, list)) {
        path[strcspn(path, "\n")] = 0;
        if (!path[0])
            continue;
        struct rt_gguf g;
        char err[512];
        memset(err, 0x55, sizeof err);
        if (rt_gguf_read(&g, path, err, sizeof err) != 0) {
            refused++;
            if (!memchr(err, 0, sizeof err) || strncmp(err, path, strlen(path)) != 0 || !strstr(err, ": "))
                violation(path, "a refusal without \"path: reason\"", 0, 0);
            continue;
        }
        accepted++;
        check(path, &g);
        rt_gguf_free(&g);
    }
    fclose(list);
    printf("accepted %ld refused %ld violations %ld\n", accepted, refused, violations);
    return violations ? 1 : 0;
}
