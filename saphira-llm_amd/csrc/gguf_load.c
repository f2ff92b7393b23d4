/*
 * gguf_load.c -- a BitNet-b1.58 GGUF v3 file onto the device.
 *
 * Reads the container in place (the caller's mapping; FORMAT.md:9-117 of
 * saphira-llm), applies the same acceptance rules and returns the same
 * statuses as the reference's parser and loader (src/gguf.c:488-700,
 * src/forward.c:269-455), and hands the tensors it found to
 * sllm_gfx950_model_upload. Nothing is copied on the host: tensor pointers
 * point into the image, and only a small index of the metadata is
 * allocated.
 */
#define _POSIX_C_SOURCE 200809L

#include "shim_internal.h"

#include <saphira_amd/sllm_gfx950_decode.h>

#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* limits of include/saphira_llm/gguf.h:31-35 and src/forward.c:45 */
#define GG_MAX_TENSORS (1u << 20)
#define GG_MAX_KV      (1u << 22)
#define GG_MAX_STRING  (1u << 30)
#define GG_MAX_ARRAY   (1u << 28)
#define GG_MAX_LAYERS  64

enum { VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STR, VT_ARR, VT_U64, VT_I64,
       VT_F64, VT_COUNT };
static const uint8_t k_vt_size[VT_COUNT] = { 1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8 };

enum { T_F32 = 0, T_F16 = 1, T_I2S = 36 };

/* Tensor types of the format (FORMAT.md:78-112): elements per block and
 * bytes per block; 0 / 0 marks a known type whose size is not a fixed block
 * (its extent cannot be checked), -1 an unknown number. */
static int type_traits(uint32_t type, uint32_t *blck, uint32_t *bytes) {
    static const struct { uint32_t t, blck, bytes; } k[] = {
        { 0, 1, 4 }, { 1, 1, 2 }, { 30, 1, 2 }, { 8, 32, 34 }, { 2, 32, 18 }, { 12, 256, 144 },
        { 14, 256, 210 }, { 36, 1, 0 }, { 3, 32, 20 }, { 6, 32, 22 }, { 7, 32, 24 }, { 10, 256, 84 },
        { 11, 256, 110 }, { 13, 256, 176 }, { 20, 32, 18 }, { 22, 256, 82 }, { 23, 256, 136 },
        { 24, 1, 1 }, { 25, 1, 2 }, { 26, 1, 4 }, { 27, 1, 8 }, { 28, 1, 8 }, { 34, 256, 54 },
        { 35, 256, 66 }, { 39, 32, 17 }, { 40, 64, 36 }, { 37, 0, 0 }, { 41, 0, 0 }, { 42, 0, 0 },
    };
    for (size_t i = 0; i < sizeof k / sizeof k[0]; ++i) {
        if (k[i].t == type) { *blck = k[i].blck; *bytes = k[i].bytes; return 0; }
    }
    return -1;
}

typedef struct gg_kv {
    const char    *key;
    uint64_t       key_len;    /* up to the first NUL: the reference keeps keys as C strings */
    uint32_t       type, arr_type;
    uint64_t       n;          /* array length, 1 for scalars */
    const uint8_t *val;        /* first element (scalars and fixed-size arrays) */
} gg_kv;

typedef struct gg_tensor {
    const char    *name;
    uint64_t       name_len;   /* up to the first NUL, as for keys */
    uint32_t       n_dims, type;
    uint64_t       ne[4];
    uint64_t       offset, nbytes;
    int            sized;
    const uint8_t *data;
} gg_tensor;

typedef struct gg_file {
    const uint8_t *base;
    size_t         size, pos;
    gg_kv         *kv;
    uint64_t       n_kv;
    gg_tensor     *t;
    uint64_t       n_t;
} gg_file;

static int need(gg_file *f, uint64_t n) { return n <= f->size - f->pos; }

static int rd_u32(gg_file *f, uint32_t *v) {
    if (!need(f, 4)) return 0;
    memcpy(v, f->base + f->pos, 4);
    f->pos += 4;
    return 1;
}

static int rd_u64(gg_file *f, uint64_t *v) {
    if (!need(f, 8)) return 0;
    memcpy(v, f->base + f->pos, 8);
    f->pos += 8;
    return 1;
}

static int rd_str(gg_file *f, const char **s, uint64_t *len) {
    if (!rd_u64(f, len) || *len > GG_MAX_STRING || !need(f, *len)) return 0;
    *s = (const char *) (f->base + f->pos);
    f->pos += *len;
    return 1;
}

/* length of a file string as a C string (the reference copies each string
 * and NUL-terminates it, so comparisons stop at an embedded NUL) */
static uint64_t c_len(const char *s, uint64_t len) {
    const void *z = memchr(s, 0, len);
    return z != NULL ? (uint64_t) ((const char *) z - s) : len;
}

static int read_kv(gg_file *f, gg_kv *kv) {
    uint32_t vt;
    if (!rd_str(f, &kv->key, &kv->key_len) || !rd_u32(f, &vt)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
    kv->key_len = c_len(kv->key, kv->key_len);
    if (vt >= VT_COUNT) return SLLM_GFX950_ERR_GGUF_TYPE;
    kv->type = vt;
    kv->arr_type = vt;
    kv->n = 1;
    if (vt == VT_ARR) {
        uint32_t at;
        uint64_t n;
        if (!rd_u32(f, &at) || !rd_u64(f, &n)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        if (at >= VT_COUNT || at == VT_ARR) return SLLM_GFX950_ERR_GGUF_TYPE;
        if (n > GG_MAX_ARRAY) return SLLM_GFX950_ERR_TOO_LARGE;
        kv->arr_type = at;
        kv->n = n;
        kv->val = f->base + f->pos;
        if (at == VT_STR) {
            if (n > f->size / 8) return SLLM_GFX950_ERR_TOO_LARGE;
            for (uint64_t i = 0; i < n; ++i) {
                const char *s;
                uint64_t l;
                if (!rd_str(f, &s, &l)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
            }
            return 0;
        }
        const uint64_t bytes = n * k_vt_size[at];
        if (!need(f, bytes)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        f->pos += bytes;
        return 0;
    }
    kv->val = f->base + f->pos;
    if (vt == VT_STR) {
        const char *s;
        uint64_t l;
        if (!rd_str(f, &s, &l)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        return 0;
    }
    if (!need(f, k_vt_size[vt])) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
    f->pos += k_vt_size[vt];
    return 0;
}

/* Keys seen so far, open addressing on FNV-1a: each key is checked against
 * the earlier ones as soon as it is read, so a duplicate is reported before
 * anything later in the file is looked at, as src/gguf.c:541-557 does. */
typedef struct key_set {
    uint32_t *slot;            /* kv index + 1, 0 = empty */
    uint64_t  mask;
} key_set;

static uint64_t key_hash(const char *s, uint64_t n) {
    uint64_t h = 1469598103934665603ull;
    for (uint64_t i = 0; i < n; ++i) h = (h ^ (uint8_t) s[i]) * 1099511628211ull;
    return h;
}

/* 1 if kv i repeats an earlier key, else records it */
static int key_seen(key_set *ks, const gg_kv *kv, uint32_t i) {
    for (uint64_t j = key_hash(kv[i].key, kv[i].key_len) & ks->mask;; j = (j + 1) & ks->mask) {
        if (ks->slot[j] == 0) {
            ks->slot[j] = i + 1;
            return 0;
        }
        const gg_kv *o = &kv[ks->slot[j] - 1];
        if (o->key_len == kv[i].key_len && memcmp(o->key, kv[i].key, o->key_len) == 0) return 1;
    }
}

static int cmp_offset(const void *a, const void *b) {
    const gg_tensor *x = *(const gg_tensor *const *) a, *y = *(const gg_tensor *const *) b;
    return x->offset < y->offset ? -1 : (x->offset > y->offset ? 1 : 0);
}

static const gg_kv *find_kv(const gg_file *f, const char *key) {
    const size_t len = strlen(key);
    for (uint64_t i = 0; i < f->n_kv; ++i) {
        if (f->kv[i].key_len == len && memcmp(f->kv[i].key, key, len) == 0) return &f->kv[i];
    }
    return NULL;
}

static const gg_tensor *find_tensor(const gg_file *f, const char *name) {
    const size_t len = strlen(name);
    for (uint64_t i = 0; i < f->n_t; ++i) {
        if (f->t[i].name_len == len && memcmp(f->t[i].name, name, len) == 0) return &f->t[i];
    }
    return NULL;
}

/* The container (src/gguf.c:488-700): header, metadata, tensor table,
 * alignment, extents inside the blob and not overlapping. */
static int parse(gg_file *f) {
    uint32_t version;
    if (f->size < 4) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
    if (memcmp(f->base, "GGUF", 4) != 0) return SLLM_GFX950_ERR_GGUF_MAGIC;
    f->pos = 4;
    if (!rd_u32(f, &version)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
    if (version != 3) return SLLM_GFX950_ERR_GGUF_VERSION;
    if (!rd_u64(f, &f->n_t) || !rd_u64(f, &f->n_kv)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
    if (f->n_t > GG_MAX_TENSORS || f->n_kv > GG_MAX_KV) return SLLM_GFX950_ERR_TOO_LARGE;
    /* A metadata entry takes at least 12 bytes of the file (key length and
     * value type) and a tensor entry at least 32 (name length, rank, one
     * dimension, type, offset), so a header that declares more than the file
     * can hold fails on a truncated read before it reaches entry
     * size / 12 + 1 (size / 32 + 1): the index is sized by that, not by the
     * declared counts. */
    const uint64_t kv_cap = f->n_kv < f->size / 12 + 1 ? f->n_kv : f->size / 12 + 1;
    const uint64_t t_cap = f->n_t < f->size / 32 + 1 ? f->n_t : f->size / 32 + 1;
    uint64_t slots = 2;
    while (slots < 2 * kv_cap) slots <<= 1;
    key_set ks = { calloc(slots, sizeof *ks.slot), slots - 1 };
    f->kv = calloc(kv_cap ? kv_cap : 1, sizeof *f->kv);
    f->t = calloc(t_cap ? t_cap : 1, sizeof *f->t);
    if (ks.slot == NULL || f->kv == NULL || f->t == NULL) {
        free(ks.slot);
        return SLLM_GFX950_ERR_NOMEM;
    }
    for (uint64_t i = 0; i < f->n_kv; ++i) {
        if (i == kv_cap) {
            free(ks.slot);
            return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        }
        int st = read_kv(f, &f->kv[i]);
        if (st == 0 && key_seen(&ks, f->kv, (uint32_t) i)) st = SLLM_GFX950_ERR_GGUF_KEYDUP;
        if (st != 0) {
            free(ks.slot);
            return st;
        }
    }
    free(ks.slot);
    for (uint64_t i = 0; i < f->n_t; ++i) {
        if (i == t_cap) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        gg_tensor *t = &f->t[i];
        if (!rd_str(f, &t->name, &t->name_len) || !rd_u32(f, &t->n_dims)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        t->name_len = c_len(t->name, t->name_len);
        if (t->n_dims == 0 || t->n_dims > 4) return SLLM_GFX950_ERR_GGUF_TENSOR;
        uint64_t nelem = 1;
        for (uint32_t d = 0; d < t->n_dims; ++d) {
            if (!rd_u64(f, &t->ne[d])) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
            if (t->ne[d] == 0 || nelem > UINT64_MAX / t->ne[d]) return SLLM_GFX950_ERR_GGUF_TENSOR;
            nelem *= t->ne[d];
        }
        for (uint32_t d = t->n_dims; d < 4; ++d) t->ne[d] = 1;
        if (!rd_u32(f, &t->type) || !rd_u64(f, &t->offset)) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
        uint32_t blck, bytes;
        if (type_traits(t->type, &blck, &bytes) != 0) return SLLM_GFX950_ERR_GGUF_TENSOR;
        /* A tensor whose size cannot be computed (a type of no fixed block,
         * or an element count that is not whole blocks) is kept but not
         * placed: its extent is not checked and it has no data
         * (src/gguf.c:613-627). */
        if (t->type == T_I2S) {                 /* four codes per byte, then the 32-byte tail */
            t->sized = nelem % 4 == 0;
            t->nbytes = t->sized ? nelem / 4 + 32 : 0;
        } else if (blck != 0 && nelem % blck == 0) {
            t->nbytes = nelem / blck * bytes;
            t->sized = 1;
        }
    }
    uint64_t align = 32;
    const gg_kv *a = find_kv(f, "general.alignment");
    if (a != NULL && a->type == VT_U32) {
        uint32_t v;
        memcpy(&v, a->val, 4);
        if (v == 0 || (v & (v - 1)) != 0) return SLLM_GFX950_ERR_GGUF_ALIGNMENT;
        align = v;
    }
    const uint64_t data_at = ((uint64_t) f->pos + align - 1) & ~(align - 1);
    if (data_at > f->size) return SLLM_GFX950_ERR_GGUF_TRUNCATED;
    const uint64_t blob = f->size - data_at;
    for (uint64_t i = 0; i < f->n_t; ++i) {
        gg_tensor *t = &f->t[i];
        if (!t->sized) continue;
        if (t->offset > blob || t->nbytes > blob - t->offset) return SLLM_GFX950_ERR_GGUF_LAYOUT;
        t->data = f->base + data_at + t->offset;
    }
    if (f->n_t > 1) {
        const gg_tensor **order = malloc(f->n_t * sizeof *order);
        if (order == NULL) return SLLM_GFX950_ERR_NOMEM;
        uint64_t n = 0;
        for (uint64_t i = 0; i < f->n_t; ++i) {
            if (f->t[i].sized) order[n++] = &f->t[i];
        }
        qsort(order, n, sizeof *order, cmp_offset);
        int overlap = 0;
        for (uint64_t i = 1; i < n && !overlap; ++i) overlap = order[i - 1]->offset + order[i - 1]->nbytes > order[i]->offset;
        free(order);
        if (overlap) return SLLM_GFX950_ERR_GGUF_LAYOUT;
    }
    return 0;
}

/* an unsigned 32-bit key as src/gguf.c:874-892 reads one (a scalar of that
 * type or the first element of such an array, in range) */
static int kv_u32(const gg_file *f, const char *key, uint32_t *out) {
    const gg_kv *kv = find_kv(f, key);
    if (kv == NULL || kv->arr_type != VT_U32 || kv->n < 1) return -1;
    memcpy(out, kv->val, 4);
    return 0;
}

static int kv_f32(const gg_file *f, const char *key, float *out) {
    const gg_kv *kv = find_kv(f, key);
    if (kv == NULL || kv->arr_type != VT_F32 || kv->n < 1) return -1;
    memcpy(out, kv->val, 4);
    return 0;
}

/* a tensor of the given type and rank (src/forward.c:269-316), and for I2_S
 * a contracted width that is a whole number of 128-element blocks */
static const gg_tensor *need_tensor(const gg_file *f, const char *name, uint32_t type, uint32_t n_dims) {
    const gg_tensor *t = find_tensor(f, name);
    if (t == NULL || t->type != type || t->n_dims != n_dims || !t->sized) return NULL;
    if (type == T_I2S && t->ne[0] % 128 != 0) return NULL;
    return t;
}

/* The model's metadata and tensors (src/forward.c:318-455): the
 * architecture, ten hyper-parameters, then every tensor by name, type, rank
 * and shape. layers must hold 64 entries. */
static int describe(const gg_file *f, sllm_gfx950_model_desc *d, sllm_gfx950_layer_desc *layers) {
    const gg_kv *arch = find_kv(f, "general.architecture");
    static const char want[] = "bitnet-b1.58";
    if (arch == NULL || arch->type != VT_STR) return SLLM_GFX950_ERR_ARCH;
    uint64_t alen;
    memcpy(&alen, arch->val, 8);
    alen = c_len((const char *) arch->val + 8, alen);
    if (alen != sizeof want - 1 || memcmp(arch->val + 8, want, alen) != 0) return SLLM_GFX950_ERR_ARCH;
    uint32_t u[8];
    static const char *keys[8] = {
        "bitnet-b1.58.block_count", "bitnet-b1.58.embedding_length", "bitnet-b1.58.feed_forward_length",
        "bitnet-b1.58.attention.head_count", "bitnet-b1.58.attention.head_count_kv",
        "bitnet-b1.58.rope.dimension_count", "bitnet-b1.58.context_length", "bitnet-b1.58.vocab_size",
    };
    for (int i = 0; i < 8; ++i) {
        if (kv_u32(f, keys[i], &u[i]) != 0) return SLLM_GFX950_ERR_KV_MISSING;
    }
    memset(d, 0, sizeof *d);
    if (kv_f32(f, "bitnet-b1.58.attention.layer_norm_rms_epsilon", &d->eps) != 0 ||
        kv_f32(f, "bitnet-b1.58.rope.freq_base", &d->rope_base) != 0) {
        return SLLM_GFX950_ERR_KV_MISSING;
    }
    d->n_layer = (int32_t) u[0]; d->n_embd = (int32_t) u[1]; d->n_ff = (int32_t) u[2];
    d->n_head = (int32_t) u[3]; d->n_head_kv = (int32_t) u[4]; d->n_rot = (int32_t) u[5];
    d->n_vocab = (int32_t) u[7];
    if (d->n_layer <= 0 || d->n_layer > GG_MAX_LAYERS || d->n_embd <= 0 || d->n_head <= 0 ||
        d->n_head_kv <= 0 || d->n_head % d->n_head_kv != 0 || d->n_ff <= 0 || d->n_vocab <= 0 ||
        d->n_embd % d->n_head != 0 || d->n_rot > d->n_embd / d->n_head) {
        return SLLM_GFX950_ERR_TENSOR_SHAPE;
    }
    const uint64_t e = (uint64_t) d->n_embd, ff = (uint64_t) d->n_ff, v = (uint64_t) d->n_vocab;
    const uint64_t gqa = e / (uint64_t) d->n_head * (uint64_t) d->n_head_kv;
    const gg_tensor *t = need_tensor(f, "token_embd.weight", T_F16, 2);
    if (t == NULL || t->ne[0] != e || t->ne[1] != v) return SLLM_GFX950_ERR_TENSOR_SHAPE;
    d->tok_embd = (const uint16_t *) t->data;
    t = need_tensor(f, "output_norm.weight", T_F32, 1);
    if (t == NULL || t->ne[0] != e) return SLLM_GFX950_ERR_TENSOR_SHAPE;
    d->output_norm = (const float *) t->data;
    static const struct { const char *name; int i2s; int k; int rows; } spec[11] = {
        /* k / rows: 0 n_embd, 1 n_embd_gqa, 2 n_ff */
        { "attn_q", 1, 0, 0 }, { "attn_k", 1, 0, 1 }, { "attn_v", 1, 0, 1 }, { "attn_output", 1, 0, 0 },
        { "ffn_gate", 1, 0, 2 }, { "ffn_up", 1, 0, 2 }, { "ffn_down", 1, 2, 0 },
        { "attn_norm", 0, 0, 0 }, { "attn_sub_norm", 0, 0, 0 }, { "ffn_norm", 0, 0, 0 }, { "ffn_sub_norm", 0, 2, 0 },
    };
    const uint64_t dim[3] = { e, gqa, ff };
    for (int32_t il = 0; il < d->n_layer; ++il) {
        const void *p[11];
        for (int s = 0; s < 11; ++s) {
            char name[128];
            snprintf(name, sizeof name, "blk.%d.%s.weight", (int) il, spec[s].name);
            t = need_tensor(f, name, spec[s].i2s ? T_I2S : T_F32, spec[s].i2s ? 2 : 1);
            if (t == NULL || t->ne[0] != dim[spec[s].k] || (spec[s].i2s && t->ne[1] != dim[spec[s].rows])) {
                return SLLM_GFX950_ERR_TENSOR_SHAPE;
            }
            p[s] = t->data;
        }
        layers[il] = (sllm_gfx950_layer_desc) { p[0], p[1], p[2], p[3], p[4], p[5], p[6],
                                                p[7], p[8], p[9], p[10] };
    }
    d->layers = layers;
    return 0;
}

int sllm_gfx950_gguf_describe(const void *image, size_t size, sllm_gfx950_model_desc *desc,
                              sllm_gfx950_layer_desc *layers) {
    if (image == NULL || desc == NULL || layers == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "gguf: NULL argument");
    gg_file f = { .base = image, .size = size };
    int st = parse(&f);
    if (st == 0) st = describe(&f, desc, layers);
    free(f.kv);
    free(f.t);
    if (st != 0) return sllm_shim_fail(st, "gguf: rejected with status %d", st);
    return SLLM_GFX950_OK;
}

int sllm_gfx950_model_load_gguf(const void *image, size_t size, sllm_gfx950_model **out) {
    if (out == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "gguf: NULL out pointer");
    *out = NULL;
    sllm_gfx950_layer_desc *layers = calloc(GG_MAX_LAYERS, sizeof *layers);
    if (layers == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_NOMEM, "gguf: host");
    sllm_gfx950_model_desc d;
    int st = sllm_gfx950_gguf_describe(image, size, &d, layers);
    if (st == SLLM_GFX950_OK) st = sllm_gfx950_model_upload(&d, out);
    free(layers);
    return st;
}

int sllm_gfx950_model_load_gguf_file(const char *path, sllm_gfx950_model **out) {
    if (path == NULL || out == NULL) return sllm_shim_fail(SLLM_GFX950_ERR_ARG, "gguf: NULL argument");
    *out = NULL;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return sllm_shim_fail(SLLM_GFX950_ERR_IO, "gguf: cannot open %s", path);
    struct stat sb;
    if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode)) {
        close(fd);
        return sllm_shim_fail(SLLM_GFX950_ERR_IO, "gguf: %s is not a regular file", path);
    }
    if (sb.st_size <= 0) {
        close(fd);
        return sllm_shim_fail(SLLM_GFX950_ERR_GGUF_TRUNCATED, "gguf: %s is empty", path);
    }
    void *map = mmap(NULL, (size_t) sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (map == MAP_FAILED) return sllm_shim_fail(SLLM_GFX950_ERR_IO, "gguf: cannot map %s", path);
    const int st = sllm_gfx950_model_load_gguf(map, (size_t) sb.st_size, out);
    munmap(map, (size_t) sb.st_size);
    return st;
}
