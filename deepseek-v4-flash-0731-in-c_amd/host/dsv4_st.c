/* dsv4_st.c - checkpoint index: every tensor of every *.safetensors shard in
 * a directory, found by name, read by byte span. It feeds the HBM loader
 * (csrc/dsv4_load.hip), which reads each layer once into device memory.
 *
 * Contract kept from the reference reader (src/io/k3_st.h:66-99,
 * src/io/k3_st.c:203-470):
 *  - a shard is [u64 little-endian N][N bytes of JSON header][data]; a
 *    tensor's data_offsets are relative to the end of the header;
 *  - shards are the directory's *.safetensors files sorted by name (shard
 *    index = position in that order); tensors keep discovery order (shard,
 *    then header order); "__metadata__" and unknown keys are skipped;
 *  - dtypes U8, I8, I64, BF16, F16, F32, F8_E4M3, F8_E8M0; rank at most 4;
 *    shape [] is a scalar (one element);
 *  - a tensor whose byte span differs from numel * elemsize, or that ends
 *    past the end of its file, or a name seen twice (in any shards) makes the
 *    open fail;
 *  - JSON string escapes are decoded (\uXXXX keeps ASCII, anything else
 *    becomes '?'), names are at most 511 bytes.
 * Stricter than the reference: negative dimensions or offsets, an end offset
 * before the start, and numbers that overflow int64 are rejected.
 * Errors return a DSV4G_E* code with the message in dsv4g_last_error().
 */
#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#include "dsv4_gpu.h"

int dsv4g_fail(int code, const char *fmt, ...); /* csrc/dsv4_runtime.hip */

#define NAME_MAX_BYTES 512 /* including the terminating NUL */
#define POOL_BLOCK (1u << 20)

/* Names live in fixed blocks that never move, so a tensor's name pointer is
 * valid from the moment it is stored until dsv4g_st_close. */
typedef struct PoolBlock {
    struct PoolBlock *next;
    size_t used, cap;
    char data[];
} PoolBlock;

struct DSV4GSt {
    int nshard;
    int *fd;
    char **path;
    DSV4GTensor *t;
    int nt, cap;
    int32_t *slot; /* open addressing, -1 = empty */
    uint64_t mask;
    PoolBlock *pool;
};

static const struct {
    const char *name;
    int dtype, size;
} DTYPES[] = {
    {"U8", DSV4G_DT_U8, 1},           {"I8", DSV4G_DT_I8, 1},
    {"I64", DSV4G_DT_I64, 8},         {"BF16", DSV4G_DT_BF16, 2},
    {"F16", DSV4G_DT_F16, 2},         {"F32", DSV4G_DT_F32, 4},
    {"F8_E4M3", DSV4G_DT_F8_E4M3, 1}, {"F8_E8M0", DSV4G_DT_F8_E8M0, 1},
};

int dsv4g_st_elemsize(int dtype)
{
    for (size_t i = 0; i < sizeof DTYPES / sizeof DTYPES[0]; i++)
        if (DTYPES[i].dtype == dtype) return DTYPES[i].size;
    return 0;
}

const char *dsv4g_st_dtype_name(int dtype)
{
    for (size_t i = 0; i < sizeof DTYPES / sizeof DTYPES[0]; i++)
        if (DTYPES[i].dtype == dtype) return DTYPES[i].name;
    return "UNKNOWN";
}

int64_t dsv4g_st_numel(const DSV4GTensor *t)
{
    int64_t n = 1;
    for (int i = 0; i < t->ndim; i++) n *= t->shape[i];
    return n;
}

/* 64-bit FNV-1a (Fowler, Noll, Vo): every byte of the name enters the hash,
 * which matters because checkpoint names share long prefixes. */
static uint64_t name_hash(const char *s)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (; *s; s++) h = (h ^ (unsigned char)*s) * 0x100000001b3ull;
    return h;
}

static const char *pool_add(DSV4GSt *st, const char *s, size_t n)
{
    PoolBlock *b = st->pool;
    if (!b || b->cap - b->used < n + 1) {
        size_t cap = n + 1 > POOL_BLOCK ? n + 1 : POOL_BLOCK;
        b = (PoolBlock *)malloc(sizeof *b + cap);
        if (!b) return NULL;
        b->next = st->pool;
        b->used = 0;
        b->cap = cap;
        st->pool = b;
    }
    char *p = b->data + b->used;
    memcpy(p, s, n);
    p[n] = '\0';
    b->used += n + 1;
    return p;
}

/* ------------------------------------------------------- header parsing -- */
typedef struct {
    const char *p, *end;
    const char *path;
} Cursor;

static void skip_ws(Cursor *c)
{
    while (c->p < c->end && (unsigned char)*c->p <= ' ') c->p++;
}

/* consume c if it is the next non-blank character */
static int take(Cursor *c, char ch)
{
    skip_ws(c);
    if (c->p < c->end && *c->p == ch) {
        c->p++;
        return 1;
    }
    return 0;
}

static int hex_val(char h)
{
    if (h >= '0' && h <= '9') return h - '0';
    if (h >= 'a' && h <= 'f') return h - 'a' + 10;
    if (h >= 'A' && h <= 'F') return h - 'A' + 10;
    return -1;
}

/* A JSON string into out[cap] (NUL-terminated). 0 on success. */
static int read_string(Cursor *c, char *out, size_t cap, size_t *len)
{
    skip_ws(c);
    if (c->p >= c->end || *c->p != '"') return -1;
    c->p++;
    size_t n = 0;
    for (;;) {
        if (c->p >= c->end) return -1;
        char ch = *c->p++;
        if (ch == '"') break;
        if (ch == '\\') {
            if (c->p >= c->end) return -1;
            char e = *c->p++;
            switch (e) {
            case 'b': ch = '\b'; break;
            case 'f': ch = '\f'; break;
            case 'n': ch = '\n'; break;
            case 'r': ch = '\r'; break;
            case 't': ch = '\t'; break;
            case 'u': {
                if (c->end - c->p < 4) return -1;
                unsigned v = 0;
                for (int i = 0; i < 4; i++) {
                    int d = hex_val(*c->p++);
                    if (d < 0) return -1;
                    v = v * 16u + (unsigned)d;
                }
                ch = v < 128 ? (char)v : '?';
                break;
            }
            default: ch = e; /* \" \\ \/ */
            }
        }
        if (n + 1 >= cap) return -1;
        out[n++] = ch;
    }
    out[n] = '\0';
    if (len) *len = n;
    return 0;
}

static int read_int(Cursor *c, int64_t *v)
{
    skip_ws(c);
    int neg = 0;
    if (c->p < c->end && (*c->p == '-' || *c->p == '+')) neg = *c->p++ == '-';
    if (c->p >= c->end || *c->p < '0' || *c->p > '9') return -1;
    uint64_t a = 0;
    while (c->p < c->end && *c->p >= '0' && *c->p <= '9') {
        if (a > (uint64_t)(INT64_MAX - 9) / 10) return -1;
        a = a * 10 + (uint64_t)(*c->p++ - '0');
    }
    *v = neg ? -(int64_t)a : (int64_t)a;
    return 0;
}

/* Step over one JSON value of any shape (the __metadata__ object, keys the
 * index does not use). */
static int skip_value(Cursor *c)
{
    skip_ws(c);
    if (c->p >= c->end) return -1;
    int depth = 0;
    do {
        if (c->p >= c->end) return -1;
        char ch = *c->p;
        if (ch == '"') {
            c->p++;
            while (c->p < c->end && *c->p != '"') c->p += (*c->p == '\\') ? 2 : 1;
            if (c->p >= c->end) return -1;
            c->p++;
        } else if (ch == '{' || ch == '[') {
            depth++;
            c->p++;
        } else if (ch == '}' || ch == ']') {
            if (depth == 0) return -1;
            depth--;
            c->p++;
        } else if (depth == 0) {
            /* bare scalar: up to the next delimiter */
            while (c->p < c->end && *c->p != ',' && *c->p != '}' && *c->p != ']') c->p++;
            return 0;
        } else {
            c->p++;
        }
    } while (depth > 0);
    return 0;
}

static int bad(const Cursor *c, const char *what)
{
    return dsv4g_fail(DSV4G_EIO, "%s: %s", c->path, what);
}

/* One header entry {"dtype":..., "shape":[...], "data_offsets":[a,b], ...}. */
static int read_entry(Cursor *c, const char *name, DSV4GTensor *t, int64_t *o0, int64_t *o1)
{
    int have_dtype = 0, have_off = 0;
    char key[NAME_MAX_BYTES];
    if (!take(c, '{')) return bad(c, "a tensor entry is not an object");
    for (int first = 1;; first = 0) {
        if (take(c, '}')) break;
        if (!first && !take(c, ',')) return bad(c, "expected ',' in a tensor entry");
        if (take(c, '}')) break;
        if (read_string(c, key, sizeof key, NULL) || !take(c, ':'))
            return bad(c, "bad key in a tensor entry");
        if (!strcmp(key, "dtype")) {
            char dv[32];
            size_t dl;
            if (read_string(c, dv, sizeof dv, &dl)) return bad(c, "bad dtype value");
            t->dtype = DSV4G_DT_UNKNOWN;
            for (size_t i = 0; i < sizeof DTYPES / sizeof DTYPES[0]; i++)
                if (!strcmp(dv, DTYPES[i].name)) t->dtype = DTYPES[i].dtype;
            if (t->dtype == DSV4G_DT_UNKNOWN)
                return dsv4g_fail(DSV4G_EIO, "%s: unsupported dtype '%s' on %s", c->path, dv,
                                  name);
            have_dtype = 1;
        } else if (!strcmp(key, "shape")) {
            t->ndim = 0;
            if (!take(c, '[')) return bad(c, "shape is not an array");
            if (!take(c, ']')) {
                for (;;) {
                    int64_t d;
                    if (read_int(c, &d) || d < 0) return bad(c, "bad shape dimension");
                    if (t->ndim == 4)
                        return dsv4g_fail(DSV4G_EIO, "%s: %s has rank > 4", c->path, name);
                    t->shape[t->ndim++] = d;
                    if (take(c, ',')) continue;
                    if (take(c, ']')) break;
                    return bad(c, "bad shape array");
                }
            }
        } else if (!strcmp(key, "data_offsets")) {
            if (!take(c, '[') || read_int(c, o0) || !take(c, ',') || read_int(c, o1) ||
                !take(c, ']'))
                return bad(c, "bad data_offsets");
            have_off = 1;
        } else if (skip_value(c)) {
            return bad(c, "bad value in a tensor entry");
        }
    }
    if (!have_dtype || !have_off)
        return dsv4g_fail(DSV4G_EIO, "%s: %s is missing dtype or data_offsets", c->path, name);
    return 0;
}

static int push_tensor(DSV4GSt *st, const DSV4GTensor *t)
{
    if (st->nt == st->cap) {
        int cap = st->cap ? st->cap * 2 : 1024;
        DSV4GTensor *nt = (DSV4GTensor *)realloc(st->t, (size_t)cap * sizeof *nt);
        if (!nt) return dsv4g_fail(DSV4G_EIO, "out of host memory indexing tensors");
        st->t = nt;
        st->cap = cap;
    }
    st->t[st->nt++] = *t;
    return 0;
}

static int pread_all(int fd, void *buf, int64_t n, int64_t off, int64_t *got_out)
{
    int64_t got = 0;
    while (got < n) {
        ssize_t r = pread(fd, (char *)buf + got, (size_t)(n - got), (off_t)(off + got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) break;
        got += r;
    }
    if (got_out) *got_out = got;
    return got == n ? 0 : -1;
}

static int index_shard(DSV4GSt *st, int shard)
{
    const char *path = st->path[shard];
    int fd = open(path, O_RDONLY);
    if (fd < 0) return dsv4g_fail(DSV4G_EIO, "cannot open %s: %s", path, strerror(errno));
    st->fd[shard] = fd;

    struct stat sb;
    if (fstat(fd, &sb)) return dsv4g_fail(DSV4G_EIO, "cannot stat %s", path);
    const int64_t fsize = (int64_t)sb.st_size;
    unsigned char lb[8];
    if (fsize < 8 || pread_all(fd, lb, 8, 0, NULL))
        return dsv4g_fail(DSV4G_EIO, "%s is too short for a header length", path);
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; i--) hlen = hlen << 8 | lb[i];
    if (hlen == 0 || hlen > (uint64_t)(fsize - 8))
        return dsv4g_fail(DSV4G_EIO, "%s header length %llu is impossible (file %lld bytes)",
                          path, (unsigned long long)hlen, (long long)fsize);

    char *json = (char *)malloc(hlen + 1);
    if (!json) return dsv4g_fail(DSV4G_EIO, "out of host memory reading %s", path);
    if (pread_all(fd, json, (int64_t)hlen, 8, NULL)) {
        free(json);
        return dsv4g_fail(DSV4G_EIO, "short read of the %s header", path);
    }
    json[hlen] = '\0';
    const int64_t base = 8 + (int64_t)hlen;

    Cursor c = {json, json + hlen, path};
    char name[NAME_MAX_BYTES];
    int rc = 0;
    if (!take(&c, '{')) {
        rc = bad(&c, "header is not a JSON object");
        goto out;
    }
    for (int first = 1;; first = 0) {
        if (take(&c, '}')) break;
        if (!first && !take(&c, ',')) {
            rc = bad(&c, "expected ',' between header entries");
            goto out;
        }
        if (take(&c, '}')) break; /* trailing comma */
        size_t nlen;
        if (read_string(&c, name, sizeof name, &nlen)) {
            rc = dsv4g_fail(DSV4G_EIO, "%s: bad tensor name near byte %ld", path,
                            (long)(c.p - json));
            goto out;
        }
        if (!take(&c, ':')) {
            rc = bad(&c, "expected ':' after a tensor name");
            goto out;
        }
        if (!strcmp(name, "__metadata__")) {
            if (skip_value(&c)) {
                rc = bad(&c, "bad __metadata__ value");
                goto out;
            }
            continue;
        }
        DSV4GTensor t;
        memset(&t, 0, sizeof t);
        int64_t o0 = 0, o1 = 0;
        if ((rc = read_entry(&c, name, &t, &o0, &o1))) goto out;
        if (o0 < 0 || o1 < o0) {
            rc = dsv4g_fail(DSV4G_EIO, "%s: %s has data_offsets [%lld, %lld]", path, name,
                            (long long)o0, (long long)o1);
            goto out;
        }
        /* the byte span must be exactly what the shape and dtype imply */
        int64_t want = dsv4g_st_elemsize(t.dtype);
        for (int i = 0; i < t.ndim; i++) {
            if (t.shape[i] && want > INT64_MAX / t.shape[i]) {
                rc = dsv4g_fail(DSV4G_EIO, "%s: %s shape overflows", path, name);
                goto out;
            }
            want *= t.shape[i];
        }
        t.off = base + o0;
        t.nbytes = o1 - o0;
        t.shard = shard;
        if (t.nbytes != want) {
            rc = dsv4g_fail(DSV4G_EIO, "%s: %s spans %lld bytes but shape implies %lld", path,
                            name, (long long)t.nbytes, (long long)want);
            goto out;
        }
        if (o1 > fsize - base) {
            rc = dsv4g_fail(DSV4G_EIO, "%s: %s ends past EOF", path, name);
            goto out;
        }
        if (!(t.name = pool_add(st, name, nlen)) || (rc = push_tensor(st, &t))) {
            if (!rc) rc = dsv4g_fail(DSV4G_EIO, "out of host memory indexing tensors");
            goto out;
        }
    }
out:
    free(json);
    return rc;
}

static int cmp_path(const void *a, const void *b)
{
    return strcmp(*(char *const *)a, *(char *const *)b);
}

void dsv4g_st_close(DSV4GSt *st)
{
    if (!st) return;
    for (int i = 0; i < st->nshard; i++) {
        if (st->fd && st->fd[i] >= 0) close(st->fd[i]);
        if (st->path) free(st->path[i]);
    }
    free(st->fd);
    free(st->path);
    free(st->t);
    free(st->slot);
    while (st->pool) {
        PoolBlock *n = st->pool->next;
        free(st->pool);
        st->pool = n;
    }
    free(st);
}

int dsv4g_st_open(DSV4GSt **out, const char *dir)
{
    if (!out || !dir) return dsv4g_fail(DSV4G_EINVAL, "dsv4g_st_open: NULL argument");
    *out = NULL;
    DSV4GSt *st = (DSV4GSt *)calloc(1, sizeof *st);
    if (!st) return dsv4g_fail(DSV4G_EIO, "out of host memory");
    int rc = 0, cap = 0;

    DIR *d = opendir(dir);
    if (!d) {
        free(st);
        return dsv4g_fail(DSV4G_EIO, "cannot open directory %s", dir);
    }
    static const char SUFFIX[] = ".safetensors";
    const size_t sl = sizeof SUFFIX - 1;
    for (struct dirent *e; (e = readdir(d));) {
        size_t n = strlen(e->d_name);
        if (n < sl || strcmp(e->d_name + n - sl, SUFFIX)) continue;
        if (st->nshard == cap) {
            cap = cap ? cap * 2 : 64;
            char **np = (char **)realloc(st->path, (size_t)cap * sizeof *np);
            if (!np) {
                rc = dsv4g_fail(DSV4G_EIO, "out of host memory");
                break;
            }
            st->path = np;
        }
        size_t len = strlen(dir) + n + 2;
        if (!(st->path[st->nshard] = (char *)malloc(len))) {
            rc = dsv4g_fail(DSV4G_EIO, "out of host memory");
            break;
        }
        memcpy(st->path[st->nshard], dir, strlen(dir));
        st->path[st->nshard][strlen(dir)] = '/';
        memcpy(st->path[st->nshard] + strlen(dir) + 1, e->d_name, n + 1);
        st->nshard++;
    }
    closedir(d);
    if (!rc && st->nshard == 0) rc = dsv4g_fail(DSV4G_EIO, "no .safetensors files in %s", dir);
    if (rc) {
        dsv4g_st_close(st);
        return rc;
    }
    /* readdir order is arbitrary: sort so shard numbers are stable */
    qsort(st->path, (size_t)st->nshard, sizeof *st->path, cmp_path);

    st->fd = (int *)malloc((size_t)st->nshard * sizeof(int));
    if (!st->fd) {
        dsv4g_st_close(st);
        return dsv4g_fail(DSV4G_EIO, "out of host memory");
    }
    for (int i = 0; i < st->nshard; i++) st->fd[i] = -1;
    for (int i = 0; i < st->nshard; i++)
        if ((rc = index_shard(st, i))) {
            dsv4g_st_close(st);
            return rc;
        }

    /* hash index at load factor below one half */
    uint64_t nslot = 1024;
    while (nslot < 2 * (uint64_t)st->nt) nslot <<= 1;
    st->slot = (int32_t *)malloc(nslot * sizeof(int32_t));
    if (!st->slot) {
        dsv4g_st_close(st);
        return dsv4g_fail(DSV4G_EIO, "out of host memory");
    }
    memset(st->slot, 0xff, nslot * sizeof(int32_t));
    st->mask = nslot - 1;
    for (int i = 0; i < st->nt; i++) {
        uint64_t j = name_hash(st->t[i].name) & st->mask;
        for (; st->slot[j] >= 0; j = (j + 1) & st->mask) {
            if (!strcmp(st->t[st->slot[j]].name, st->t[i].name)) {
                rc = dsv4g_fail(DSV4G_EIO, "duplicate tensor name %s", st->t[i].name);
                dsv4g_st_close(st);
                return rc;
            }
        }
        st->slot[j] = i;
    }
    *out = st;
    return 0;
}

const DSV4GTensor *dsv4g_st_find(const DSV4GSt *st, const char *name)
{
    if (!st || !name || !st->slot) return NULL;
    for (uint64_t j = name_hash(name) & st->mask; st->slot[j] >= 0; j = (j + 1) & st->mask)
        if (!strcmp(st->t[st->slot[j]].name, name)) return &st->t[st->slot[j]];
    return NULL;
}

int dsv4g_st_count(const DSV4GSt *st) { return st ? st->nt : 0; }

const DSV4GTensor *dsv4g_st_tensor(const DSV4GSt *st, int i)
{
    return st && i >= 0 && i < st->nt ? &st->t[i] : NULL;
}

int dsv4g_st_nshard(const DSV4GSt *st) { return st ? st->nshard : 0; }

const char *dsv4g_st_shard_path(const DSV4GSt *st, int shard)
{
    return st && shard >= 0 && shard < st->nshard ? st->path[shard] : NULL;
}

int64_t dsv4g_st_read_range(const DSV4GSt *st, int shard, int64_t off, int64_t nbytes,
                            void *buf)
{
    if (!st || shard < 0 || shard >= st->nshard || off < 0 || nbytes < 0) {
        dsv4g_fail(DSV4G_EINVAL, "dsv4g_st_read_range: bad shard %d or span", shard);
        return 0;
    }
    int64_t got;
    if (pread_all(st->fd[shard], buf, nbytes, off, &got))
        dsv4g_fail(DSV4G_EIO, "short read on %s at +%lld", st->path[shard],
                   (long long)(off + got));
    return got;
}

int64_t dsv4g_st_read(const DSV4GSt *st, const DSV4GTensor *t, void *buf)
{
    if (!st || !t) return 0;
    return dsv4g_st_read_range(st, t->shard, t->off, t->nbytes, buf);
}

/* IEEE binary16 -> binary32: exact (every half is a float). */
static float half_to_float(uint16_t h)
{
    const int e = h >> 10 & 0x1f;
    const int m = h & 0x3ff;
    union { uint32_t u; float f; } v;
    if (e == 0x1f) {
        v.u = (uint32_t)(h & 0x8000) << 16 | 0x7f800000u | (uint32_t)m << 13;
        return v.f;
    }
    /* value = (e ? 1024 + m : m) * 2^(max(e,1) - 25); both factors exact */
    v.u = (uint32_t)((e ? e : 1) - 25 + 127) << 23;
    const float mag = (float)(e ? 1024 + m : m) * v.f;
    return (h & 0x8000) ? -mag : mag;
}

#define WIDEN_CHUNK (1 << 20)

int64_t dsv4g_st_read_f32(const DSV4GSt *st, const DSV4GTensor *t, float *out)
{
    if (!st || !t) return 0;
    const int64_t n = dsv4g_st_numel(t);
    if (t->dtype == DSV4G_DT_F32) return dsv4g_st_read(st, t, out) / 4;
    const int esz = dsv4g_st_elemsize(t->dtype);
    if (esz == 0) return 0;
    unsigned char *raw = (unsigned char *)malloc(WIDEN_CHUNK);
    if (!raw) return 0;
    const int64_t per = WIDEN_CHUNK / esz;
    int64_t done = 0;
    while (done < n) {
        const int64_t k = n - done < per ? n - done : per;
        if (dsv4g_st_read_range(st, t->shard, t->off + done * esz, k * esz, raw) != k * esz)
            break;
        float *o = out + done;
        for (int64_t i = 0; i < k; i++) {
            switch (t->dtype) {
            case DSV4G_DT_BF16: {
                uint16_t b;
                memcpy(&b, raw + 2 * i, 2);
                union { uint32_t u; float f; } v = {(uint32_t)b << 16};
                o[i] = v.f;
                break;
            }
            case DSV4G_DT_F16: {
                uint16_t b;
                memcpy(&b, raw + 2 * i, 2);
                o[i] = half_to_float(b);
                break;
            }
            case DSV4G_DT_I64: {
                int64_t q;
                memcpy(&q, raw + 8 * i, 8);
                o[i] = (float)q;
                break;
            }
            default: o[i] = (float)raw[i]; /* byte dtypes: the raw code */
            }
        }
        done += k;
    }
    free(raw);
    return done;
}
