/* k3x_store.c - safetensors shards indexed by tensor name, and routed experts read as
 * byte runs (include/k3x_store.h).  Host code only: POSIX files and pread.
 *
 * Follows the reference's reader and expert loader (src/io/k3_st.{h,c}, k3_load.{h,c}):
 * the same file format, tensor naming, validation and contiguous-run read; the parser,
 * index and reads are this file's own.
 */
#define _GNU_SOURCE
#include "k3x_internal.h"
#include "../../include/k3x_store.h"

#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

typedef struct {
    char           *name;
    k3x_tensor_info t;
} st_ent;

struct k3x_store {
    int       nshard;        /* shard files opened (descriptors in fd[0 .. nshard-1]) */
    int       npath;
    int      *fd;
    char    **path;
    int64_t  *fsize;
    st_ent   *ent;
    int       n, cap;
    int32_t  *slot;          /* open-addressed index into ent, -1 empty */
    uint32_t  nslot;         /* a power of two */
};

/* ------------------------------------------------------------------ reads */
/* n bytes at off into buf, in pieces of at most 1 GiB; the count read (short at EOF). */
static int64_t read_at(int fd, void *buf, int64_t n, int64_t off)
{
    int64_t got = 0;
    while (got < n) {
        const int64_t want = n - got > ((int64_t)1 << 30) ? ((int64_t)1 << 30) : n - got;
        const ssize_t r = pread(fd, (char *)buf + got, (size_t)want, (off_t)(off + got));
        if (r < 0) {
            if (errno == EINTR) continue;
            return -1;
        }
        if (r == 0) break;
        got += r;
    }
    return got;
}

/* ------------------------------------------------------------------ JSON header */
typedef struct {
    const char *p, *end;
} jscan;

static void j_ws(jscan *j)
{
    while (j->p < j->end && (*j->p == ' ' || *j->p == '\t' || *j->p == '\n' || *j->p == '\r'))
        j->p++;
}

static int j_eat(jscan *j, char c)
{
    j_ws(j);
    if (j->p < j->end && *j->p == c) { j->p++; return 1; }
    return 0;
}

static int hexval(char h)
{
    return h >= '0' && h <= '9' ? h - '0' : h >= 'a' && h <= 'f' ? h - 'a' + 10
         : h >= 'A' && h <= 'F' ? h - 'A' + 10 : -1;
}

/* Four hex digits of a \u escape. */
static int j_hex4(jscan *j, unsigned *v)
{
    if (j->end - j->p < 4) return 0;
    unsigned x = 0;
    for (int k = 0; k < 4; k++) {
        const int h = hexval(*j->p++);
        if (h < 0) return 0;
        x = x * 16 + (unsigned)h;
    }
    *v = x;
    return 1;
}

/* A JSON string into out (cap bytes, NUL-terminated): bytes copied as they are, escapes
 * decoded (\uXXXX to UTF-8, surrogate pairs joined).  0 on a malformed or too long one. */
static int j_str(jscan *j, char *out, size_t cap)
{
    if (!j_eat(j, '"')) return 0;
    size_t n = 0;
    while (j->p < j->end && *j->p != '"') {
        unsigned char b[4];
        int nb = 1;
        const char c = *j->p++;
        if (c != '\\') {
            b[0] = (unsigned char)c;
        } else {
            if (j->p >= j->end) return 0;
            const char e = *j->p++;
            unsigned cp = 0;
            switch (e) {
            case '"': case '\\': case '/': cp = (unsigned char)e; break;
            case 'b': cp = '\b'; break;
            case 'f': cp = '\f'; break;
            case 'n': cp = '\n'; break;
            case 'r': cp = '\r'; break;
            case 't': cp = '\t'; break;
            case 'u': {
                if (!j_hex4(j, &cp)) return 0;
                if (cp >= 0xD800 && cp < 0xDC00) {          /* a surrogate pair */
                    unsigned lo;
                    if (j->end - j->p < 2 || j->p[0] != '\\' || j->p[1] != 'u') return 0;
                    j->p += 2;
                    if (!j_hex4(j, &lo) || lo < 0xDC00 || lo >= 0xE000) return 0;
                    cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                }
                break;
            }
            default: return 0;
            }
            if (cp < 0x80) { b[0] = (unsigned char)cp; }
            else if (cp < 0x800) { b[0] = (unsigned char)(0xC0 | (cp >> 6)); b[1] = (unsigned char)(0x80 | (cp & 63)); nb = 2; }
            else if (cp < 0x10000) { b[0] = (unsigned char)(0xE0 | (cp >> 12)); b[1] = (unsigned char)(0x80 | ((cp >> 6) & 63)); b[2] = (unsigned char)(0x80 | (cp & 63)); nb = 3; }
            else { b[0] = (unsigned char)(0xF0 | (cp >> 18)); b[1] = (unsigned char)(0x80 | ((cp >> 12) & 63)); b[2] = (unsigned char)(0x80 | ((cp >> 6) & 63)); b[3] = (unsigned char)(0x80 | (cp & 63)); nb = 4; }
        }
        if (n + (size_t)nb >= cap) return 0;
        memcpy(out + n, b, (size_t)nb);
        n += (size_t)nb;
    }
    if (!j_eat(j, '"')) return 0;
    out[n] = '\0';
    return 1;
}

static int j_int(jscan *j, int64_t *v)
{
    j_ws(j);
    int neg = 0;
    if (j->p < j->end && *j->p == '-') { neg = 1; j->p++; }
    if (j->p >= j->end || *j->p < '0' || *j->p > '9') return 0;
    int64_t x = 0;
    while (j->p < j->end && *j->p >= '0' && *j->p <= '9') {
        if (x > (INT64_MAX - 9) / 10) return 0;
        x = x * 10 + (*j->p++ - '0');
    }
    *v = neg ? -x : x;
    return 1;
}

/* Any value, nesting tracked, strings skipped whole. */
static int j_skip(jscan *j)
{
    j_ws(j);
    if (j->p >= j->end) return 0;
    const char c = *j->p;
    if (c == '"') {
        j->p++;
        while (j->p < j->end && *j->p != '"') j->p += (*j->p == '\\') ? 2 : 1;
        if (j->p >= j->end) return 0;
        j->p++;
        return 1;
    }
    if (c == '{' || c == '[') {
        const char close = c == '{' ? '}' : ']';
        j->p++;
        if (j_eat(j, close)) return 1;
        for (;;) {
            if (c == '{') {
                if (!j_skip(j) || !j_eat(j, ':')) return 0;
            }
            if (!j_skip(j)) return 0;
            if (j_eat(j, ',')) continue;
            return j_eat(j, close);
        }
    }
    /* number, true, false, null */
    const char *s = j->p;
    while (j->p < j->end && *j->p != ',' && *j->p != '}' && *j->p != ']' && *j->p != ' ' &&
           *j->p != '\n' && *j->p != '\r' && *j->p != '\t')
        j->p++;
    return j->p > s;
}

static int dtype_of(const char *s)
{
    if (!strcmp(s, "U8")) return K3X_DT_U8;
    if (!strcmp(s, "BF16")) return K3X_DT_BF16;
    if (!strcmp(s, "F16")) return K3X_DT_F16;
    if (!strcmp(s, "F32")) return K3X_DT_F32;
    return K3X_DT_UNKNOWN;
}

static int dtype_size(int d) { return d == K3X_DT_U8 ? 1 : (d == K3X_DT_F32 ? 4 : 2); }

/* ------------------------------------------------------------------ index */
static uint64_t name_hash(const char *s)
{
    uint64_t h = 0x243F6A8885A308D3ull;
    for (; *s; s++) {
        h = (h + (unsigned char)*s) * 0x9E3779B97F4A7C15ull;
        h ^= h >> 29;
    }
    return h;
}

static int index_build(k3x_store *s)
{
    uint32_t ns = 16;
    while (ns < (uint32_t)s->n * 2u + 16u) ns <<= 1;
    s->slot = (int32_t *)malloc((size_t)ns * sizeof(int32_t));
    if (!s->slot) return K3X_E_NOMEM;
    s->nslot = ns;
    for (uint32_t i = 0; i < ns; i++) s->slot[i] = -1;
    for (int i = 0; i < s->n; i++) {
        uint32_t h = (uint32_t)name_hash(s->ent[i].name) & (ns - 1);
        while (s->slot[h] >= 0) {
            if (!strcmp(s->ent[s->slot[h]].name, s->ent[i].name)) {
                fprintf(stderr, "k3x_store: tensor %s appears twice\n", s->ent[i].name);
                return K3X_E_ARG;
            }
            h = (h + 1) & (ns - 1);
        }
        s->slot[h] = i;
    }
    return 0;
}

static const st_ent *lookup(const k3x_store *s, const char *name)
{
    if (!s || !name || !s->slot) return NULL;
    uint32_t h = (uint32_t)name_hash(name) & (s->nslot - 1);
    while (s->slot[h] >= 0) {
        const st_ent *e = &s->ent[s->slot[h]];
        if (!strcmp(e->name, name)) return e;
        h = (h + 1) & (s->nslot - 1);
    }
    return NULL;
}

static int add_entry(k3x_store *s, const char *name, const k3x_tensor_info *t)
{
    if (s->n == s->cap) {
        const int nc = s->cap ? s->cap * 2 : 256;
        st_ent *ne = (st_ent *)realloc(s->ent, (size_t)nc * sizeof(st_ent));
        if (!ne) return K3X_E_NOMEM;
        s->ent = ne;
        s->cap = nc;
    }
    char *dup = strdup(name);
    if (!dup) return K3X_E_NOMEM;
    s->ent[s->n].name = dup;
    s->ent[s->n].t = *t;
    s->n++;
    return 0;
}

/* Parse one shard's header and add its tensors. */
static int scan_shard(k3x_store *s, int shard)
{
    const int fd = s->fd[shard];
    unsigned char lenb[8];
    if (read_at(fd, lenb, 8, 0) != 8) return K3X_E_ARG;
    uint64_t hl = 0;
    for (int i = 7; i >= 0; i--) hl = (hl << 8) | lenb[i];
    if (hl < 2 || hl > ((uint64_t)1 << 30) || (int64_t)(8 + hl) > s->fsize[shard]) {
        fprintf(stderr, "k3x_store: %s: bad header length\n", s->path[shard]);
        return K3X_E_ARG;
    }
    char *hdr = (char *)malloc((size_t)hl);
    if (!hdr) return K3X_E_NOMEM;
    int rc = K3X_E_ARG;
    if (read_at(fd, hdr, (int64_t)hl, 8) != (int64_t)hl) goto out;
    const int64_t data0 = 8 + (int64_t)hl;
    jscan j = {hdr, hdr + hl};
    char name[4096], key[64], dt[32];
    if (!j_eat(&j, '{')) goto bad;
    if (j_eat(&j, '}')) { rc = 0; goto out; }
    for (;;) {
        if (!j_str(&j, name, sizeof name) || !j_eat(&j, ':')) goto bad;
        if (!strcmp(name, "__metadata__")) {
            if (!j_skip(&j)) goto bad;
        } else {
            k3x_tensor_info t;
            memset(&t, 0, sizeof t);
            t.shard = shard;
            int have_dt = 0, have_shape = 0, have_off = 0;
            int64_t b0 = 0, b1 = 0;
            if (!j_eat(&j, '{')) goto bad;
            if (!j_eat(&j, '}')) {
                for (;;) {
                    if (!j_str(&j, key, sizeof key) || !j_eat(&j, ':')) goto bad;
                    if (!strcmp(key, "dtype")) {
                        if (!j_str(&j, dt, sizeof dt)) goto bad;
                        t.dtype = dtype_of(dt);
                        if (!t.dtype) {
                            fprintf(stderr, "k3x_store: %s: dtype %s of %s not supported\n",
                                    s->path[shard], dt, name);
                            goto out;
                        }
                        have_dt = 1;
                    } else if (!strcmp(key, "shape")) {
                        if (!j_eat(&j, '[')) goto bad;
                        if (!j_eat(&j, ']')) {
                            for (;;) {
                                int64_t v;
                                if (t.ndim == 4 || !j_int(&j, &v) || v < 0) goto bad;
                                t.shape[t.ndim++] = v;
                                if (j_eat(&j, ',')) continue;
                                if (!j_eat(&j, ']')) goto bad;
                                break;
                            }
                        }
                        have_shape = 1;
                    } else if (!strcmp(key, "data_offsets")) {
                        if (!j_eat(&j, '[') || !j_int(&j, &b0) || !j_eat(&j, ',') ||
                            !j_int(&j, &b1) || !j_eat(&j, ']'))
                            goto bad;
                        have_off = 1;
                    } else if (!j_skip(&j)) {
                        goto bad;
                    }
                    if (j_eat(&j, ',')) continue;
                    if (!j_eat(&j, '}')) goto bad;
                    break;
                }
            }
            if (!have_dt || !have_shape || !have_off || b0 < 0 || b1 < b0) goto bad;
            /* every product and sum checked: a crafted header must not wrap around */
            int64_t numel = 1, want = 0, end = 0;
            int ovf = 0;
            for (int d = 0; d < t.ndim; d++) ovf |= __builtin_mul_overflow(numel, t.shape[d], &numel);
            ovf |= __builtin_mul_overflow(numel, (int64_t)dtype_size(t.dtype), &want);
            ovf |= __builtin_add_overflow(data0, b0, &t.off);
            t.nbytes = b1 - b0;
            ovf |= __builtin_add_overflow(t.off, t.nbytes, &end);
            if (ovf || want != t.nbytes || end > s->fsize[shard]) {
                fprintf(stderr, "k3x_store: %s: %s has %lld bytes for its shape or leaves the file\n",
                        s->path[shard], name, (long long)t.nbytes);
                goto out;
            }
            if ((rc = add_entry(s, name, &t))) goto out;
            rc = K3X_E_ARG;
        }
        if (j_eat(&j, ',')) continue;
        if (!j_eat(&j, '}')) goto bad;
        break;
    }
    rc = 0;
    goto out;
bad:
    fprintf(stderr, "k3x_store: %s: malformed header\n", s->path[shard]);
    rc = K3X_E_ARG;
out:
    free(hdr);
    return rc;
}

static int cmp_names(const void *a, const void *b)
{
    return strcmp(*(char *const *)a, *(char *const *)b);
}

int k3x_store_open(const char *dir, k3x_store **out)
{
    if (!dir || !out) return K3X_E_ARG;
    *out = NULL;
    k3x_store *s = (k3x_store *)calloc(1, sizeof *s);
    if (!s) return K3X_E_NOMEM;
    int rc = 0, cap = 0;
    DIR *d = opendir(dir);
    if (!d) { free(s); return K3X_E_ARG; }
    const struct dirent *de;
    while ((de = readdir(d))) {
        const size_t l = strlen(de->d_name);
        if (l <= 12 || strcmp(de->d_name + l - 12, ".safetensors")) continue;
        if (s->npath == cap) {
            cap = cap ? 2 * cap : 16;
            char **np = (char **)realloc(s->path, (size_t)cap * sizeof(char *));
            if (!np) { rc = K3X_E_NOMEM; break; }
            s->path = np;
        }
        char *p = (char *)malloc(strlen(dir) + l + 2);
        if (!p) { rc = K3X_E_NOMEM; break; }
        sprintf(p, "%s/%s", dir, de->d_name);
        s->path[s->npath++] = p;
    }
    closedir(d);
    if (!rc && s->npath == 0) rc = K3X_E_ARG;
    if (!rc) {
        qsort(s->path, (size_t)s->npath, sizeof(char *), cmp_names);
        s->fd = (int *)malloc((size_t)s->npath * sizeof(int));
        s->fsize = (int64_t *)calloc((size_t)s->npath, sizeof(int64_t));
        if (!s->fd || !s->fsize) rc = K3X_E_NOMEM;
    }
    for (int i = 0; !rc && i < s->npath; i++) {
        const int fd = open(s->path[i], O_RDONLY | O_CLOEXEC);
        if (fd < 0) { rc = K3X_E_ARG; break; }
        s->fd[i] = fd;
        s->nshard = i + 1;
        struct stat stt;
        if (fstat(fd, &stt)) { rc = K3X_E_ARG; break; }
        s->fsize[i] = (int64_t)stt.st_size;
        rc = scan_shard(s, i);
    }
    if (!rc) rc = index_build(s);
    if (rc) {
        k3x_store_close(s);
        return rc;
    }
    *out = s;
    return 0;
}

void k3x_store_close(k3x_store *s)
{
    if (!s) return;
    for (int i = 0; i < s->nshard; i++) close(s->fd[i]);
    for (int i = 0; i < s->npath; i++) free(s->path[i]);
    for (int i = 0; i < s->n; i++) free(s->ent[i].name);
    free(s->ent);
    free(s->fd);
    free(s->fsize);
    free(s->path);
    free(s->slot);
    free(s);
}

int k3x_store_count(const k3x_store *s) { return s ? s->n : 0; }
int k3x_store_shards(const k3x_store *s) { return s ? s->nshard : 0; }

int k3x_store_find(const k3x_store *s, const char *name, k3x_tensor_info *info)
{
    const st_ent *e = lookup(s, name);
    if (!e) return K3X_E_ARG;
    if (info) *info = e->t;
    return 0;
}

int64_t k3x_store_read(const k3x_store *s, const char *name, void *buf, int64_t cap)
{
    const st_ent *e = lookup(s, name);
    if (!e || !buf || cap < e->t.nbytes) return K3X_E_ARG;
    const int64_t got = read_at(s->fd[e->t.shard], buf, e->t.nbytes, e->t.off);
    return got == e->t.nbytes ? got : K3X_E_ARG;
}

/* ------------------------------------------------------------------ experts */
#define EXPERT_NAME "language_model.model.layers.%d.block_sparse_moe.experts.%d.w%d.%s"

int k3x_store_expert_ref(const k3x_store *s, int layer, int expert, k3x_expert_ref *r)
{
    if (!s || !r) return K3X_E_ARG;
    memset(r, 0, sizeof *r);
    r->layer = layer;
    r->expert = expert;
    const st_ent *pk[3], *sc[3];
    char name[256];
    for (int i = 0; i < 3; i++) {
        snprintf(name, sizeof name, EXPERT_NAME, layer, expert, i + 1, "weight_packed");
        pk[i] = lookup(s, name);
        snprintf(name, sizeof name, EXPERT_NAME, layer, expert, i + 1, "weight_scale");
        sc[i] = lookup(s, name);
        if (!pk[i] || !sc[i]) {
            fprintf(stderr, "k3x_store: layer %d expert %d: w%d is missing\n", layer, expert, i + 1);
            return K3X_E_ARG;
        }
        const k3x_tensor_info *p = &pk[i]->t, *q = &sc[i]->t;
        if (p->dtype != K3X_DT_U8 || q->dtype != K3X_DT_U8 || p->ndim != 2 || q->ndim != 2 ||
            p->shape[0] != q->shape[0]) {
            fprintf(stderr, "k3x_store: layer %d expert %d: w%d is not a U8 [rows][...] pair\n",
                    layer, expert, i + 1);
            return K3X_E_ARG;
        }
        /* one E8M0 scale per 32 elements; anything else would apply every scale after the
         * first to the wrong elements */
        if (q->shape[1] * 32 != p->shape[1] * 2) {
            fprintf(stderr, "k3x_store: layer %d expert %d: w%d has %lld scales for %lld "
                            "elements, not one per 32\n", layer, expert, i + 1,
                    (long long)q->shape[1], (long long)(p->shape[1] * 2));
            return K3X_E_ARG;
        }
        if (q->shard != p->shard || p->shard != pk[0]->t.shard) {
            fprintf(stderr, "k3x_store: layer %d expert %d spans shards\n", layer, expert);
            return K3X_E_ARG;
        }
        r->m[i].rows = (int)p->shape[0];
        r->m[i].pcols = (int)p->shape[1];
        r->m[i].scols = (int)q->shape[1];
        r->m[i].p_bytes = p->nbytes;
        r->m[i].s_bytes = q->nbytes;
    }
    r->shard = pk[0]->t.shard;
    const st_ent *all[6] = {pk[0], sc[0], pk[1], sc[1], pk[2], sc[2]};
    int64_t lo = all[0]->t.off, hi = 0, sum = 0;
    for (int i = 0; i < 6; i++) {
        const int64_t a = all[i]->t.off, b = a + all[i]->t.nbytes;
        lo = a < lo ? a : lo;
        hi = b > hi ? b : hi;
        sum += all[i]->t.nbytes;
    }
    r->contiguous = (hi - lo == sum);
    r->off = lo;
    r->nbytes = sum;
    int64_t o = 0;
    for (int i = 0; i < 3; i++) {
        if (r->contiguous) {
            r->m[i].p_off = pk[i]->t.off - lo;
            r->m[i].s_off = sc[i]->t.off - lo;
        } else {                         /* packed in canonical order, six reads */
            r->m[i].p_off = o; o += r->m[i].p_bytes;
            r->m[i].s_off = o; o += r->m[i].s_bytes;
        }
    }
    return 0;
}

int64_t k3x_store_expert_load(const k3x_store *s, const k3x_expert_ref *r, unsigned char *buf)
{
    if (!s || !r || !buf || r->shard < 0 || r->shard >= s->nshard) return K3X_E_ARG;
    const int fd = s->fd[r->shard];
    if (r->contiguous) {
        const int64_t got = read_at(fd, buf, r->nbytes, r->off);
        return got == r->nbytes ? got : K3X_E_ARG;
    }
    char name[256];
    int64_t got = 0;
    for (int i = 0; i < 3; i++) {
        for (int k = 0; k < 2; k++) {
            snprintf(name, sizeof name, EXPERT_NAME, r->layer, r->expert, i + 1,
                     k ? "weight_scale" : "weight_packed");
            const st_ent *e = lookup(s, name);
            if (!e) return K3X_E_ARG;
            const int64_t dst = k ? r->m[i].s_off : r->m[i].p_off;
            const int64_t n = read_at(fd, buf + dst, e->t.nbytes, e->t.off);
            if (n != e->t.nbytes) return K3X_E_ARG;
            got += n;
        }
    }
    return got;
}

/* ------------------------------------------------------------------ supplier */
typedef struct {
    k3x_expert_src base;          /* first member: get() casts back */
    k3x_store     *s;
    unsigned char *buf;
    int64_t        cap;
    long           fetches;
    int            inter, width;  /* the layer's expert shape, or 0: not checked */
} store_src;

/* w1/w3 [I][X] and w2 [X][I] with one scale per 32 elements, for some I and X (or the
 * supplier's I and X when it has them) */
static int expert_shape_ok(const store_src *ss, const k3x_expert_ref *r)
{
    const int I = ss->inter ? ss->inter : r->m[0].rows;
    const int X = ss->width ? ss->width : r->m[0].pcols * 2;
    const int rows[3] = {I, X, I}, width[3] = {X, I, X};
    for (int i = 0; i < 3; i++)
        if (r->m[i].rows != rows[i] || r->m[i].pcols * 2 != width[i] ||
            r->m[i].scols * 32 != width[i])
            return 0;
    return 1;
}

static int store_get(k3x_expert_src *self, int layer, int expert, k3x_expert_q *q)
{
    store_src *ss = (store_src *)self;
    k3x_expert_ref r;
    if (k3x_store_expert_ref(ss->s, layer, expert, &r)) return -1;
    if (!expert_shape_ok(ss, &r)) {
        fprintf(stderr, "k3x_store: layer %d expert %d has matrices of the wrong shape\n",
                layer, expert);
        return -1;
    }
    if (r.nbytes > ss->cap) {
        unsigned char *nb = (unsigned char *)realloc(ss->buf, (size_t)r.nbytes);
        if (!nb) return -1;
        ss->buf = nb;
        ss->cap = r.nbytes;
    }
    if (k3x_store_expert_load(ss->s, &r, ss->buf) != r.nbytes) return -1;
    ss->fetches++;
    q->p1 = ss->buf + r.m[0].p_off; q->s1 = ss->buf + r.m[0].s_off;   /* w1: gate */
    q->p3 = ss->buf + r.m[2].p_off; q->s3 = ss->buf + r.m[2].s_off;   /* w3: up   */
    q->p2 = ss->buf + r.m[1].p_off; q->s2 = ss->buf + r.m[1].s_off;   /* w2: down */
    return 0;
}

/* getmany: the experts' byte ranges handed to the kernel's read-ahead together
 * (POSIX_FADV_WILLNEED), so that the get() calls that follow find them in the page
 * cache.  Advisory: nothing is made resident in this supplier (get() still reads), so
 * it returns 0 experts resident, or -1 when a range cannot be found. */
static int store_getmany(k3x_expert_src *self, int layer, const int *experts, int n)
{
    store_src *ss = (store_src *)self;
    char name[256];
    for (int i = 0; i < n; i++) {
        k3x_expert_ref r;
        if (k3x_store_expert_ref(ss->s, layer, experts[i], &r)) return -1;
        const int fd = ss->s->fd[r.shard];
        if (r.contiguous) {
            (void)posix_fadvise(fd, (off_t)r.off, (off_t)r.nbytes, POSIX_FADV_WILLNEED);
            continue;
        }
        for (int m = 0; m < 3; m++)
            for (int k = 0; k < 2; k++) {
                snprintf(name, sizeof name, EXPERT_NAME, layer, experts[i], m + 1,
                         k ? "weight_scale" : "weight_packed");
                const st_ent *e = lookup(ss->s, name);
                if (!e) return -1;
                (void)posix_fadvise(fd, (off_t)e->t.off, (off_t)e->t.nbytes, POSIX_FADV_WILLNEED);
            }
    }
    return 0;
}

int k3x_store_src_create_for(k3x_store *s, int moe_inter, int width, k3x_expert_src **out)
{
    if (!s || !out || moe_inter < 0 || width < 0) return K3X_E_ARG;
    store_src *ss = (store_src *)calloc(1, sizeof *ss);
    if (!ss) return K3X_E_NOMEM;
    ss->base.get = store_get;
    ss->base.getmany = store_getmany;
    ss->base.ctx = ss;
    ss->s = s;
    ss->inter = moe_inter;
    ss->width = width;
    *out = &ss->base;
    return 0;
}

int k3x_store_src_create(k3x_store *s, k3x_expert_src **out)
{
    return k3x_store_src_create_for(s, 0, 0, out);
}

void k3x_store_src_destroy(k3x_expert_src *src)
{
    if (!src) return;
    store_src *ss = (store_src *)src;
    free(ss->buf);
    free(ss);
}

long k3x_store_src_fetches(const k3x_expert_src *src)
{
    return src ? ((const store_src *)src)->fetches : 0;
}
