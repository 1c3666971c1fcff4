/* exl3c4_import.c -- routed experts of an EXL3 checkpoint (exllamav3's safetensors layout, as turboderp's conversions
 * are published) into the canonical planes this library's relayout takes: the import the reference's `exl3` quantiser
 * performs (quantizers/exl3/exl3_quant.cpp:192-256; its checkpoint reader quantizers/exl3/exl3_src.cpp). Host code,
 * load time; nothing here touches a GPU.
 *
 * A checkpoint directory holds config.json (quantization_config.quant_method "exl3"; the layer count
 * text_config.num_hidden_layers, else num_hidden_layers) and its tensors, in model.safetensors or in the shards that
 * model.safetensors.index.json's weight_map names. A safetensors file is a little-endian u64 header length, a JSON
 * header {name: {dtype, shape, data_offsets: [begin, end]}, "__metadata__": {...}} and the tensors' bytes, offsets
 * counted from the header's end. Headers are parsed once, on the first lookup that needs them (metadata only); a
 * tensor's bytes are read on demand into the caller's buffer.
 *
 * The weight blk.L.ffn_gate_up_exps.E.weight (stacked: gate rows, then up rows) is <P>.E.gate_proj and <P>.E.up_proj;
 * blk.L.ffn_down_exps.E.weight is <P>.E.down_proj; <P> is model.language_model.layers.L.mlp.experts for a trunk layer
 * and mtp.layers.0.mlp.experts for the MTP head, whose layer index is the layer count (exl3_quant.cpp:283-296). A
 * projection is trellis I16 [k/16, n/16, 16 K] (exllamav3's tile record, tk outer), suh F16 [k], svh F16 [n] and a
 * codebook marker: an I32 scalar .mul1 = 0x83DCD12D or .mcg = 0xCBAC1FED, neither meaning 3inst
 * (exl3_quant.cpp:142-178). Every refusal of the reference is kept, with its status (exl3_quant.cpp:12-20); all of a
 * weight's parts are checked before any plane is written.
 *
 * Little-endian hosts only (the bytes are taken as stored): exl3c4_ckpt_open refuses a big-endian one. */
#define _POSIX_C_SOURCE 200809L   /* strdup */
#include <errno.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "exl3c4.h"

/* ------------------------------------------------------------------ JSON: a tree in one node array */
enum { J_NULL, J_BOOL, J_NUM, J_STR, J_ARR, J_OBJ };
typedef struct JNode {
    int    kind;
    double num;
    char*  str;      /* J_STR: the value; a member: its key (kept in `key`) */
    char*  key;
    int    child, next;   /* first child and next sibling, -1 for none */
} JNode;
typedef struct Json {
    JNode* n;
    int    len, cap;
    const char *p, *end;
    int    bad;
} Json;

static int jnew(Json* j, int kind) {
    if (j->len == j->cap) {
        const int cap = j->cap ? 2 * j->cap : 256;
        JNode* m = (JNode*)realloc(j->n, (size_t)cap * sizeof *m);
        if (!m) { j->bad = 1; return -1; }
        j->n = m;
        j->cap = cap;
    }
    JNode* x = &j->n[j->len];
    memset(x, 0, sizeof *x);
    x->kind = kind;
    x->child = x->next = -1;
    return j->len++;
}
static void jskip(Json* j) {
    while (j->p < j->end && (*j->p == ' ' || *j->p == '\t' || *j->p == '\n' || *j->p == '\r')) ++j->p;
}
static void jput_utf8(char** o, unsigned cp) {
    if (cp < 0x80) *(*o)++ = (char)cp;
    else if (cp < 0x800) { *(*o)++ = (char)(0xC0 | (cp >> 6)); *(*o)++ = (char)(0x80 | (cp & 63)); }
    else {
        *(*o)++ = (char)(0xE0 | (cp >> 12));
        *(*o)++ = (char)(0x80 | ((cp >> 6) & 63));
        *(*o)++ = (char)(0x80 | (cp & 63));
    }
}
/* A string at j->p (the opening quote): a fresh NUL-terminated copy, escapes resolved (\uXXXX to UTF-8; a surrogate
 * pair's halves each as their own code point, enough for names). */
static char* jstring(Json* j) {
    if (j->p >= j->end || *j->p != '"') { j->bad = 1; return NULL; }
    ++j->p;
    const char* s = j->p;
    while (j->p < j->end && *j->p != '"') j->p += (*j->p == '\\' && j->p + 1 < j->end) ? 2 : 1;
    if (j->p >= j->end) { j->bad = 1; return NULL; }
    char* out = (char*)malloc((size_t)(j->p - s) * 3 + 1);
    if (!out) { j->bad = 1; return NULL; }
    char* o = out;
    for (const char* q = s; q < j->p; ++q) {
        if (*q != '\\') { *o++ = *q; continue; }
        ++q;
        switch (*q) {
        case 'b': *o++ = '\b'; break;
        case 'f': *o++ = '\f'; break;
        case 'n': *o++ = '\n'; break;
        case 'r': *o++ = '\r'; break;
        case 't': *o++ = '\t'; break;
        case 'u': {
            unsigned cp = 0;
            for (int i = 0; i < 4; ++i) {
                const char c = (q + 1 < j->p) ? *++q : 0;
                cp = cp * 16 + (unsigned)(c >= '0' && c <= '9' ? c - '0' : c >= 'a' && c <= 'f' ? c - 'a' + 10
                                          : c >= 'A' && c <= 'F' ? c - 'A' + 10 : (j->bad = 1, 0));
            }
            jput_utf8(&o, cp);
            break;
        }
        default: *o++ = *q; break;     /* \" \\ \/ */
        }
    }
    *o = 0;
    ++j->p;                            /* the closing quote */
    return out;
}
static int jvalue(Json* j, int depth) {
    jskip(j);
    if (j->bad || j->p >= j->end || depth > 64) { j->bad = 1; return -1; }
    const char c = *j->p;
    if (c == '{' || c == '[') {
        const int obj = c == '{';
        const int me = jnew(j, obj ? J_OBJ : J_ARR);
        if (me < 0) return -1;
        ++j->p;
        int last = -1;
        jskip(j);
        if (j->p < j->end && *j->p == (obj ? '}' : ']')) { ++j->p; return me; }
        for (;;) {
            char* key = NULL;
            if (obj) {
                jskip(j);
                key = jstring(j);
                jskip(j);
                if (j->bad || j->p >= j->end || *j->p != ':') { free(key); j->bad = 1; return -1; }
                ++j->p;
            }
            const int v = jvalue(j, depth + 1);
            if (v < 0) { free(key); return -1; }
            j->n[v].key = key;
            if (last < 0) j->n[me].child = v;
            else j->n[last].next = v;
            last = v;
            jskip(j);
            if (j->p < j->end && *j->p == ',') { ++j->p; continue; }
            if (j->p < j->end && *j->p == (obj ? '}' : ']')) { ++j->p; return me; }
            j->bad = 1;
            return -1;
        }
    }
    if (c == '"') {
        const int me = jnew(j, J_STR);
        if (me < 0) return -1;
        char* s = jstring(j);
        j->n[me].str = s;
        return j->bad ? -1 : me;
    }
    if (c == 't' || c == 'f' || c == 'n') {
        const char* w = c == 't' ? "true" : c == 'f' ? "false" : "null";
        const size_t l = strlen(w);
        if ((size_t)(j->end - j->p) < l || memcmp(j->p, w, l)) { j->bad = 1; return -1; }
        j->p += l;
        const int me = jnew(j, c == 'n' ? J_NULL : J_BOOL);
        if (me >= 0) j->n[me].num = c == 't';
        return me;
    }
    /* a number */
    char buf[64];
    size_t l = 0;
    while (j->p < j->end && l + 1 < sizeof buf && strchr("+-0123456789.eE", *j->p)) buf[l++] = *j->p++;
    buf[l] = 0;
    char* e = NULL;
    const double v = strtod(buf, &e);
    if (!l || *e) { j->bad = 1; return -1; }
    const int me = jnew(j, J_NUM);
    if (me >= 0) j->n[me].num = v;
    return me;
}
static void jfree(Json* j) {
    for (int i = 0; i < j->len; ++i) {
        free(j->n[i].str);
        free(j->n[i].key);
    }
    free(j->n);
    memset(j, 0, sizeof *j);
}
/* Parse [p, p + len): the root node (0), or -1 (malformed, or nesting deeper than 64). */
static int jparse(Json* j, const char* p, size_t len) {
    memset(j, 0, sizeof *j);
    j->p = p;
    j->end = p + len;
    const int r = jvalue(j, 0);
    jskip(j);
    if (r < 0 || j->bad || j->p != j->end) return -1;
    return r;
}
static int jget(const Json* j, int obj, const char* key) {
    if (obj < 0 || j->n[obj].kind != J_OBJ) return -1;
    for (int c = j->n[obj].child; c >= 0; c = j->n[c].next)
        if (j->n[c].key && !strcmp(j->n[c].key, key)) return c;
    return -1;
}

/* ------------------------------------------------------------------ files */
static int read_file(const char* path, char** out, size_t* len) {
    FILE* f = fopen(path, "rb");
    if (!f) return errno == ENOENT ? EXL3C4_E_NOTFOUND : EXL3C4_E_IO;
    int rc = EXL3C4_E_IO;
    char* buf = NULL;
    if (fseek(f, 0, SEEK_END) == 0) {
        const long n = ftell(f);
        if (n >= 0 && fseek(f, 0, SEEK_SET) == 0 && (buf = (char*)malloc((size_t)n + 1)) != NULL &&
            fread(buf, 1, (size_t)n, f) == (size_t)n) {
            buf[n] = 0;
            *out = buf;
            *len = (size_t)n;
            buf = NULL;
            rc = EXL3C4_OK;
        }
    }
    free(buf);
    fclose(f);
    return rc;
}

/* ------------------------------------------------------------------ the checkpoint */
typedef struct Tensor {
    char*    name;
    int      shard;        /* index into Exl3c4Ckpt.shard */
    int      known;        /* the shard's header was read and holds it */
    char     dtype[8];
    int      rank;
    int64_t  shape[8];
    uint64_t begin, end;   /* absolute byte offsets in the shard */
} Tensor;

struct Exl3c4Ckpt {
    char*           dir;
    int64_t         layers;
    char**          shard;         /* shard file names (relative to dir) */
    int*            shard_loaded;
    int             n_shard;
    Tensor*         t;             /* open-addressed by name (FNV-1a), cap a power of two */
    int64_t         cap, count;
    pthread_mutex_t mu;
};

static uint64_t fnv(const char* s) {
    uint64_t h = 1469598103934665603ull;
    for (; *s; ++s) h = (h ^ (uint8_t)*s) * 1099511628211ull;
    return h;
}
static Tensor* slot(Exl3c4Ckpt* c, const char* name) {      /* the name's slot: its entry, or the empty one */
    for (uint64_t i = fnv(name) & (uint64_t)(c->cap - 1);; i = (i + 1) & (uint64_t)(c->cap - 1))
        if (!c->t[i].name || !strcmp(c->t[i].name, name)) return &c->t[i];
}
static int grow(Exl3c4Ckpt* c) {
    if (2 * (c->count + 1) <= c->cap) return 0;
    const int64_t cap = c->cap ? 2 * c->cap : 1024;
    Tensor* old = c->t;
    const int64_t ocap = c->cap;
    c->t = (Tensor*)calloc((size_t)cap, sizeof *c->t);
    if (!c->t) { c->t = old; return -1; }
    c->cap = cap;
    for (int64_t i = 0; i < ocap; ++i)
        if (old[i].name) *slot(c, old[i].name) = old[i];
    free(old);
    return 0;
}
/* The entry of `name`, inserted (for shard `shard`, header not yet read) if new. */
static Tensor* insert(Exl3c4Ckpt* c, const char* name, int shard) {
    if (grow(c)) return NULL;
    Tensor* t = slot(c, name);
    if (!t->name) {
        if (!(t->name = strdup(name))) return NULL;
        t->shard = shard;
        ++c->count;
    }
    return t;
}
static int add_shard(Exl3c4Ckpt* c, const char* file) {
    for (int i = 0; i < c->n_shard; ++i)
        if (!strcmp(c->shard[i], file)) return i;
    char** s = (char**)realloc(c->shard, (size_t)(c->n_shard + 1) * sizeof *s);
    if (!s) return -1;
    c->shard = s;
    int* l = (int*)realloc(c->shard_loaded, (size_t)(c->n_shard + 1) * sizeof *l);
    if (!l) return -1;
    c->shard_loaded = l;
    if (!(c->shard[c->n_shard] = strdup(file))) return -1;
    c->shard_loaded[c->n_shard] = 0;
    return c->n_shard++;
}
static char* join(const char* dir, const char* file) {
    const size_t a = strlen(dir), b = strlen(file);
    char* p = (char*)malloc(a + b + 2);
    if (p) {
        memcpy(p, dir, a);
        p[a] = '/';
        memcpy(p + a + 1, file, b + 1);
    }
    return p;
}

/* Read shard i's header: every tensor it holds gets its dtype, shape and absolute offsets. */
static int load_shard(Exl3c4Ckpt* c, int i) {
    char* path = join(c->dir, c->shard[i]);
    if (!path) return EXL3C4_E_IO;
    FILE* f = fopen(path, "rb");
    free(path);
    if (!f) return errno == ENOENT ? EXL3C4_E_NOTFOUND : EXL3C4_E_IO;
    uint8_t lb[8];
    int rc = EXL3C4_E_FORMAT;
    char* hdr = NULL;
    Json j;
    memset(&j, 0, sizeof j);
    if (fread(lb, 1, 8, f) != 8) goto done;
    uint64_t hl = 0;
    for (int b = 7; b >= 0; --b) hl = (hl << 8) | lb[b];
    if (hl < 2 || hl > (256ull << 20)) goto done;                 /* a header of at most 256 MiB */
    if (!(hdr = (char*)malloc((size_t)hl))) { rc = EXL3C4_E_IO; goto done; }
    if (fread(hdr, 1, (size_t)hl, f) != hl) goto done;
    if (fseek(f, 0, SEEK_END) != 0) { rc = EXL3C4_E_IO; goto done; }
    const long fsize = ftell(f);
    const int root = jparse(&j, hdr, (size_t)hl);
    if (root < 0 || j.n[root].kind != J_OBJ) goto done;
    const uint64_t base = 8 + hl;
    for (int m = j.n[root].child; m >= 0; m = j.n[m].next) {
        const char* name = j.n[m].key;
        if (!strcmp(name, "__metadata__")) continue;
        const int dt = jget(&j, m, "dtype"), sh = jget(&j, m, "shape"), off = jget(&j, m, "data_offsets");
        if (dt < 0 || j.n[dt].kind != J_STR || strlen(j.n[dt].str) >= 8 || sh < 0 || j.n[sh].kind != J_ARR || off < 0 ||
            j.n[off].kind != J_ARR)
            goto done;
        Tensor* t = insert(c, name, i);
        if (!t) { rc = EXL3C4_E_IO; goto done; }
        if (t->shard != i) continue;                              /* the index names another shard for it */
        strcpy(t->dtype, j.n[dt].str);
        t->rank = 0;
        for (int d = j.n[sh].child; d >= 0; d = j.n[d].next) {
            if (t->rank == 8 || j.n[d].kind != J_NUM || j.n[d].num < 0) goto done;
            t->shape[t->rank++] = (int64_t)j.n[d].num;
        }
        const int b0 = j.n[off].child, b1 = b0 >= 0 ? j.n[b0].next : -1;
        if (b0 < 0 || b1 < 0 || j.n[b1].next >= 0 || j.n[b0].kind != J_NUM || j.n[b1].kind != J_NUM) goto done;
        const double o0 = j.n[b0].num, o1 = j.n[b1].num;
        if (o0 < 0 || o1 < o0 || base + (uint64_t)o1 > (uint64_t)fsize) goto done;
        t->begin = base + (uint64_t)o0;
        t->end = base + (uint64_t)o1;
        t->known = 1;
    }
    c->shard_loaded[i] = 1;
    rc = EXL3C4_OK;
done:
    jfree(&j);
    free(hdr);
    fclose(f);
    return rc;
}

void exl3c4_ckpt_close(Exl3c4Ckpt* c) {
    if (!c) return;
    for (int64_t i = 0; i < c->cap; ++i) free(c->t[i].name);
    for (int i = 0; i < c->n_shard; ++i) free(c->shard[i]);
    free(c->t);
    free(c->shard);
    free(c->shard_loaded);
    free(c->dir);
    pthread_mutex_destroy(&c->mu);
    free(c);
}

int exl3c4_ckpt_open(const char* dir, Exl3c4Ckpt** out) {
    if (!dir || !out) return EXL3C4_E_INVAL;
    *out = NULL;
    const uint16_t probe = 1;
    if (*(const uint8_t*)&probe != 1) return EXL3C4_E_FORMAT;      /* the bytes are taken as stored */
    Exl3c4Ckpt* c = (Exl3c4Ckpt*)calloc(1, sizeof *c);
    if (!c || !(c->dir = strdup(dir))) { free(c); return EXL3C4_E_IO; }
    pthread_mutex_init(&c->mu, NULL);
    c->layers = -1;
    char *text = NULL, *path = NULL;
    size_t len = 0;
    Json j;
    memset(&j, 0, sizeof j);
    int rc;
    /* config.json: an EXL3 checkpoint, and its layer count */
    if (!(path = join(dir, "config.json"))) { rc = EXL3C4_E_IO; goto fail; }
    if ((rc = read_file(path, &text, &len)) != EXL3C4_OK) { rc = rc == EXL3C4_E_NOTFOUND ? EXL3C4_E_FORMAT : rc; goto fail; }
    int root = jparse(&j, text, len);
    rc = EXL3C4_E_FORMAT;
    if (root < 0) goto fail;
    const int qm = jget(&j, jget(&j, root, "quantization_config"), "quant_method");
    if (qm < 0 || j.n[qm].kind != J_STR || strcmp(j.n[qm].str, "exl3")) goto fail;
    int nl = jget(&j, jget(&j, root, "text_config"), "num_hidden_layers");
    if (nl < 0) nl = jget(&j, root, "num_hidden_layers");
    if (nl < 0 || j.n[nl].kind != J_NUM || j.n[nl].num < 0) goto fail;
    c->layers = (int64_t)j.n[nl].num;
    jfree(&j);
    free(text);
    text = NULL;
    free(path);
    /* the tensors: the index's weight_map, or the one file */
    if (!(path = join(dir, "model.safetensors.index.json"))) { rc = EXL3C4_E_IO; goto fail; }
    rc = read_file(path, &text, &len);
    if (rc == EXL3C4_OK) {
        root = jparse(&j, text, len);
        const int wm = jget(&j, root, "weight_map");
        rc = EXL3C4_E_FORMAT;
        if (wm < 0 || j.n[wm].kind != J_OBJ) goto fail;
        for (int m = j.n[wm].child; m >= 0; m = j.n[m].next) {
            if (j.n[m].kind != J_STR || strchr(j.n[m].str, '/')) goto fail;   /* a shard beside the index */
            const int s = add_shard(c, j.n[m].str);
            if (s < 0 || !insert(c, j.n[m].key, s)) { rc = EXL3C4_E_IO; goto fail; }
        }
    } else if (rc == EXL3C4_E_NOTFOUND) {
        const int s = add_shard(c, "model.safetensors");
        if (s < 0) { rc = EXL3C4_E_IO; goto fail; }
        if ((rc = load_shard(c, s)) != EXL3C4_OK) { rc = rc == EXL3C4_E_NOTFOUND ? EXL3C4_E_FORMAT : rc; goto fail; }
    } else {
        goto fail;
    }
    jfree(&j);
    free(text);
    free(path);
    *out = c;
    return EXL3C4_OK;
fail:
    jfree(&j);
    free(text);
    free(path);
    exl3c4_ckpt_close(c);
    return rc;
}

int64_t exl3c4_ckpt_layers(const Exl3c4Ckpt* c) { return c ? c->layers : -1; }

/* Look a tensor up: 1 found (its description in *out), 0 absent, or a status < 0. */
static int find(Exl3c4Ckpt* c, const char* name, Tensor* out) {
    pthread_mutex_lock(&c->mu);
    int rc = 0;
    Tensor* t = c->cap ? slot(c, name) : NULL;
    if (t && t->name) {
        if (!c->shard_loaded[t->shard]) {
            const int s = t->shard;
            rc = load_shard(c, s);
            t = slot(c, name);                                    /* the table may have grown */
            if (rc == EXL3C4_E_NOTFOUND) rc = EXL3C4_E_FORMAT;    /* the index names a file that is not there */
        }
        if (rc == 0) {
            if (!t->known) rc = EXL3C4_E_FORMAT;                  /* the index names a shard that lacks it */
            else { *out = *t; rc = 1; }
        }
    }
    pthread_mutex_unlock(&c->mu);
    return rc;
}
static int read_tensor(const Exl3c4Ckpt* c, const Tensor* t, void* dst) {
    char* path = join(c->dir, c->shard[t->shard]);
    if (!path) return EXL3C4_E_IO;
    FILE* f = fopen(path, "rb");
    free(path);
    if (!f) return EXL3C4_E_IO;
    const size_t n = (size_t)(t->end - t->begin);
    const int ok = fseek(f, (long)t->begin, SEEK_SET) == 0 && fread(dst, 1, n, f) == n;
    fclose(f);
    return ok ? EXL3C4_OK : EXL3C4_E_IO;
}

/* ------------------------------------------------------------------ the import */
#define MUL1_MARKER 0x83DCD12Du
#define MCG_MARKER  0xCBAC1FEDu

/* blk.<L>.ffn_gate_up_exps.<E>.weight (stacked) | blk.<L>.ffn_down_exps.<E>.weight (exl3_quant.cpp:97-114) */
int exl3c4_import_parse_name(const char* s, int32_t* layer, int64_t* expert, int32_t* stacked) {
    int l = -1, at = -1;
    long long e = -1;
    if (!s) return EXL3C4_E_UNSUPPORTED;
    if (sscanf(s, "blk.%d.ffn_gate_up_exps.%lld.weight%n", &l, &e, &at) == 2 && at > 0 && s[at] == 0) {
        *stacked = 1;
    } else if (at = -1, sscanf(s, "blk.%d.ffn_down_exps.%lld.weight%n", &l, &e, &at) == 2 && at > 0 && s[at] == 0) {
        *stacked = 0;
    } else {
        return EXL3C4_E_UNSUPPORTED;
    }
    if (l < 0 || e < 0) return EXL3C4_E_UNSUPPORTED;
    *layer = l;
    *expert = e;
    return EXL3C4_OK;
}

typedef struct Part {
    const char* proj;
    int64_t     row0, rows;   /* its rows of the logical weight */
    int         up;           /* its input scales go to suh1 */
    Tensor      tr, su, sv;   /* found and checked */
} Part;

static int tensor_is(const Tensor* t, const char* dtype, int rank, const int64_t* shape) {
    if (strcmp(t->dtype, dtype) || t->rank != rank) return 0;
    for (int d = 0; d < rank; ++d)
        if (t->shape[d] != shape[d]) return 0;
    return 1;
}

/* One projection's tensors, found and checked (exl3_quant.cpp:192-247), nothing written. */
static int check_part(Exl3c4Ckpt* c, const char* prefix, Part* p, int bits, int codebook, int64_t k) {
    char name[512];
    Tensor t;
    int st;
    snprintf(name, sizeof name, "%s.%s.trellis", prefix, p->proj);
    if ((st = find(c, name, &p->tr)) <= 0) return st == 0 ? EXL3C4_E_NOTFOUND : st;
    snprintf(name, sizeof name, "%s.%s.bias", prefix, p->proj);
    if ((st = find(c, name, &t)) != 0) return st < 0 ? st : EXL3C4_E_UNSUPPORTED;
    /* the codebook: by its marker, none meaning 3inst; a marker is an I32 scalar holding the codebook's constant */
    static const struct { const char* tag; uint32_t value; int cb; } marks[2] = {
        { "mul1", MUL1_MARKER, EXL3C4_CB_MUL1 }, { "mcg", MCG_MARKER, EXL3C4_CB_MCG } };
    int cb = EXL3C4_CB_3INST, found = 0;
    for (int m = 0; m < 2; ++m) {
        snprintf(name, sizeof name, "%s.%s.%s", prefix, p->proj, marks[m].tag);
        if ((st = find(c, name, &t)) < 0) return st;
        if (st == 0) continue;
        if (strcmp(t.dtype, "I32") || t.rank != 0 || t.end - t.begin != 4) return EXL3C4_E_FORMAT;
        uint32_t v = 0;
        if ((st = read_tensor(c, &t, &v)) != EXL3C4_OK) return st;
        if (v != marks[m].value) return EXL3C4_E_FORMAT;
        cb = marks[m].cb;
        ++found;
    }
    if (found > 1) return EXL3C4_E_FORMAT;
    if (cb != codebook) return EXL3C4_E_DTYPE;
    const Tensor* tr = &p->tr;
    if (strcmp(tr->dtype, "I16") || tr->rank != 3) return EXL3C4_E_FORMAT;
    if (tr->shape[2] % 16 == 8) return EXL3C4_E_UNSUPPORTED;     /* half-integer K (exllamav3 1.5.2) */
    if (tr->shape[2] % 16 != 0) return EXL3C4_E_FORMAT;
    if (tr->shape[2] / 16 != bits) return EXL3C4_E_DTYPE;
    if (tr->shape[0] * 16 != k || tr->shape[1] * 16 != p->rows) return EXL3C4_E_SHAPE;
    if ((int64_t)(tr->end - tr->begin) != tr->shape[0] * tr->shape[1] * tr->shape[2] * 2) return EXL3C4_E_FORMAT;
    snprintf(name, sizeof name, "%s.%s.suh", prefix, p->proj);
    if ((st = find(c, name, &p->su)) <= 0) return st == 0 ? EXL3C4_E_NOTFOUND : st;
    if (!tensor_is(&p->su, "F16", 1, &k) || p->su.end - p->su.begin != (uint64_t)k * 2) return EXL3C4_E_SHAPE;
    snprintf(name, sizeof name, "%s.%s.svh", prefix, p->proj);
    if ((st = find(c, name, &p->sv)) <= 0) return st == 0 ? EXL3C4_E_NOTFOUND : st;
    if (!tensor_is(&p->sv, "F16", 1, &p->rows) || p->sv.end - p->sv.begin != (uint64_t)p->rows * 2)
        return EXL3C4_E_SHAPE;
    return EXL3C4_OK;
}

int exl3c4_import_weight(Exl3c4Ckpt* c, const char* name, int32_t bits, int32_t codebook, int64_t rows, int64_t cols,
                         uint8_t* codes, int64_t row_bytes, uint16_t* suh, uint16_t* suh1, uint16_t* svh) {
    int32_t layer, stacked;
    int64_t expert;
    int rc;
    if ((rc = exl3c4_import_parse_name(name, &layer, &expert, &stacked)) != EXL3C4_OK) return rc;
    if (!c || !codes || !suh || !svh || (stacked && !suh1)) return EXL3C4_E_INVAL;
    if (bits < 2 || bits > 8 || (codebook != EXL3C4_CB_3INST && codebook != EXL3C4_CB_MCG && codebook != EXL3C4_CB_MUL1))
        return EXL3C4_E_INVAL;
    if (rows <= 0 || cols <= 0 || rows % 128 || cols % 128 || (stacked && rows % 256)) return EXL3C4_E_SHAPE;
    if (row_bytes < cols * bits / 8) return EXL3C4_E_SHAPE;
    char prefix[160];
    if (layer < c->layers)
        snprintf(prefix, sizeof prefix, "model.language_model.layers.%d.mlp.experts.%lld", layer, (long long)expert);
    else if (layer == c->layers)
        snprintf(prefix, sizeof prefix, "mtp.layers.0.mlp.experts.%lld", (long long)expert);
    else
        return EXL3C4_E_NOTFOUND;
    Part parts[2];
    memset(parts, 0, sizeof parts);
    int np = 1;
    if (stacked) {
        parts[0].proj = "gate_proj"; parts[0].row0 = 0;        parts[0].rows = rows / 2; parts[0].up = 0;
        parts[1].proj = "up_proj";   parts[1].row0 = rows / 2; parts[1].rows = rows / 2; parts[1].up = 1;
        np = 2;
    } else {
        parts[0].proj = "down_proj"; parts[0].row0 = 0; parts[0].rows = rows; parts[0].up = 0;
    }
    for (int i = 0; i < np; ++i)                                  /* every part checked before anything is written */
        if ((rc = check_part(c, prefix, &parts[i], bits, codebook, cols)) != EXL3C4_OK) return rc;
    for (int i = 0; i < np; ++i) {
        const Part* p = &parts[i];
        if ((rc = read_tensor(c, &p->su, p->up ? suh1 : suh)) != EXL3C4_OK) return rc;
        if ((rc = read_tensor(c, &p->sv, svh + p->row0)) != EXL3C4_OK) return rc;
        uint16_t* rec = (uint16_t*)malloc((size_t)(p->tr.end - p->tr.begin));
        if (!rec) return EXL3C4_E_IO;
        if ((rc = read_tensor(c, &p->tr, rec)) == EXL3C4_OK)
            rc = exl3c4_record_to_codes(rec, p->rows, cols, bits, codes + p->row0 * row_bytes, row_bytes);
        free(rec);
        if (rc != EXL3C4_OK) return rc;
    }
    return EXL3C4_OK;
}
