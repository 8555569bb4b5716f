/* store.c -- the reference's on-disk stores (resident-manifest.json +
 * resident.bin, the sepia-index sidecar over the GGUF parts) parsed on the
 * host and uploaded straight into device memory.
 *
 * The reference parses both sidecars at load (src/sepia.c:1876-1910
 * manifest_load, :2036-2080 index_load), mmaps resident.bin and preads a
 * routed expert's three slices from its GGUF part each time the expert is
 * used, through an LRU cache (docs/container.md:238-252). On one MI355X
 * (288 GB of HBM) a layer's 256 experts fit, so a layer is uploaded whole,
 * once, and runs without host reads. The checks follow the reference's:
 * required fields, ranges inside the files, expert counts, known parts,
 * complete gate/up/down sets; failures log one line and return NULL/0
 * instead of exiting.
 *
 * Uploads stage through two pinned host buffers: the file read of one chunk
 * overlaps the DMA of the previous one, and a chunk is read by READERS
 * threads side by side (one thread's pread out of the page cache, about
 * 23 GB/s, was the slower half). The pair is allocated by the first upload
 * and kept until sepia_gpu_shutdown: the pinned allocation and release
 * cost about 1 ms per upload, and READERS threads writing pages of a
 * freshly allocated pair ran at half one thread's rate. Uploads run on the
 * library's stream and synchronize it before returning. */
#define _GNU_SOURCE 1
#include "internal.h"
#include "json.h"

#include "../../include/sepia_hip_ext.h"

#include <errno.h>
#include <fcntl.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define LOG(...) sepia_log(__VA_ARGS__)
#define STAGE_BYTES ((size_t)32 << 20)   /* each of the two pinned staging buffers */
#define READERS 4                         /* threads that read one chunk */
#define MAX_PARTS 64

/* ------------------------------------------------------------ files ----- */
static char *read_text(const char *path, size_t *len, const char *op) {
    FILE *f = fopen(path, "rb");
    if (!f) {
        LOG("%s: open %s: %s", op, path, strerror(errno));
        return NULL;
    }
    char *buf = NULL;
    size_t cap = 0, n = 0;
    for (;;) {
        if (n == cap) {
            cap = cap ? 2 * cap : (size_t)1 << 16;
            char *nb = (char *)realloc(buf, cap);
            if (!nb) {
                LOG("%s: out of host memory reading %s", op, path);
                free(buf);
                fclose(f);
                return NULL;
            }
            buf = nb;
        }
        const size_t got = fread(buf + n, 1, cap - n, f);
        n += got;
        if (got == 0) break;
    }
    const int bad = ferror(f);
    fclose(f);
    if (bad) {
        LOG("%s: read %s failed", op, path);
        free(buf);
        return NULL;
    }
    *len = n;
    return buf;
}

static SjValue *read_json(const char *path, const char *op) {
    size_t len;
    char *text = read_text(path, &len, op);
    if (!text) return NULL;
    char err[128];
    SjValue *v = sj_parse(text, len, err, sizeof err);
    free(text);
    if (!v) LOG("%s: %s: %s", op, path, err);
    return v;
}

static int file_size(const char *path, int64_t *size, const char *op) {
    struct stat st;
    if (stat(path, &st) != 0) {
        LOG("%s: stat %s: %s", op, path, strerror(errno));
        return 0;
    }
    *size = (int64_t)st.st_size;
    return 1;
}

/* dirname(path) + "/" + leaf (reference dirname_join, src/sepia.c:1823-1834). */
static char *sibling(const char *path, const char *leaf) {
    const char *slash = strrchr(path, '/');
    const size_t dl = slash ? (size_t)(slash - path) : 1;
    char *out = (char *)malloc(dl + strlen(leaf) + 2);
    if (!out) return NULL;
    memcpy(out, slash ? path : ".", dl);
    out[dl] = '/';
    strcpy(out + dl + 1, leaf);
    return out;
}

/* Required-field accessors (the reference's json_req_*, src/sepia.c:1839-1851). */
static int req_i64(const SjValue *obj, const char *key, int64_t *out, const char *what, const char *op) {
    const SjValue *v = sj_get(obj, key);
    if (!v || v->type != SJ_NUM || !v->is_int) {
        LOG("%s: %s: missing or non-integer field '%s'", op, what, key);
        return 0;
    }
    *out = v->i;
    return 1;
}
static const char *req_str(const SjValue *obj, const char *key, const char *what, const char *op) {
    const SjValue *v = sj_get(obj, key);
    if (!v || v->type != SJ_STR) {
        LOG("%s: %s: missing string field '%s'", op, what, key);
        return NULL;
    }
    return v->s;
}

/* ----------------------------------------------------- staged upload ---- */
typedef struct {
    void *host[2];
    hipEvent_t done[2];
    int used[2];
    int k;
} Stager;

static void stager_close(Stager *s) {
    hipStreamSynchronize(sepia_stream());
    for (int i = 0; i < 2; i++) {
        if (s->done[i]) hipEventDestroy(s->done[i]);
        if (s->host[i]) hipHostFree(s->host[i]);
        s->done[i] = NULL;
        s->host[i] = NULL;
    }
}

/* Two pinned staging buffers and their events; on failure whatever was
 * created is released again and 0 returned. */
static int stager_open(Stager *s, const char *op) {
    memset(s, 0, sizeof *s);
    for (int i = 0; i < 2; i++) {
        sepia_count_alloc();
        hipError_t e = hipHostMalloc(&s->host[i], STAGE_BYTES, hipHostMallocDefault);
        if (e != hipSuccess) s->host[i] = NULL;
        if (e == hipSuccess) {
            e = hipEventCreateWithFlags(&s->done[i], hipEventDisableTiming);
            if (e != hipSuccess) s->done[i] = NULL;
        }
        if (e != hipSuccess) {
            LOG("%s: staging buffers: %s", op, hipGetErrorString(e));
            stager_close(s);
            return 0;
        }
    }
    return 1;
}

/* The staging pair, held from the first upload to sepia_gpu_shutdown;
 * g_stage_lock makes uploads from different host threads take turns. */
static Stager g_stager;
static int g_stager_ready;
static pthread_mutex_t g_stage_lock = PTHREAD_MUTEX_INITIALIZER;

/* Lock the staging pair, allocating it on first use; one thread then
 * writes a byte of each page: four readers writing a freshly allocated
 * pair ran at half one reader's rate, and at twice it once its pages had
 * been written. NULL, unlocked and logged, when the allocation fails. */
static Stager *stager_acquire(const char *op) {
    pthread_mutex_lock(&g_stage_lock);
    if (!g_stager_ready) {
        if (!stager_open(&g_stager, op)) {
            pthread_mutex_unlock(&g_stage_lock);
            return NULL;
        }
        for (int i = 0; i < 2; i++)
            for (size_t b = 0; b < STAGE_BYTES; b += 4096) ((volatile uint8_t *)g_stager.host[i])[b] = 0;
        g_stager_ready = 1;
    }
    return &g_stager;
}

/* Wait for the pair's copies to finish and unlock it for the next upload. */
static void stager_release(Stager *s) {
    hipStreamSynchronize(sepia_stream());
    s->used[0] = s->used[1] = 0;
    s->k = 0;
    pthread_mutex_unlock(&g_stage_lock);
}

void sepia_store_shutdown(void) {
    pthread_mutex_lock(&g_stage_lock);
    if (g_stager_ready) stager_close(&g_stager);
    g_stager_ready = 0;
    pthread_mutex_unlock(&g_stage_lock);
}

/* One reader's share of a chunk: [off, off + n) of fd into buf. */
typedef struct {
    int fd;
    uint8_t *buf;
    int64_t off;
    size_t n, got;
    int err;   /* errno of a failed read, or -1 for an early end of file */
} ReadPart;

static void *read_part(void *arg) {
    ReadPart *p = (ReadPart *)arg;
    while (p->got < p->n) {
        const ssize_t r = pread(p->fd, p->buf + p->got, p->n - p->got, (off_t)(p->off + (int64_t)p->got));
        if (r < 0 && errno == EINTR) continue;
        if (r <= 0) {
            p->err = r < 0 ? errno : -1;
            break;
        }
        p->got += (size_t)r;
    }
    return NULL;
}

/* [off, off + n) of fd into buf by up to READERS threads; the calling
 * thread reads the first share. 0 on a failed read, logged. */
static int read_chunk(int fd, uint8_t *buf, int64_t off, size_t n, const char *path, const char *op) {
    ReadPart part[READERS];
    pthread_t th[READERS];
    int started[READERS] = {0};
    const int np = n >= (size_t)READERS << 20 ? READERS : 1;   /* small chunks: one read */
    const size_t share = (n / (size_t)np + 4095) & ~(size_t)4095;
    for (int i = 0; i < np; i++) {
        const size_t lo = (size_t)i * share < n ? (size_t)i * share : n;
        const size_t hi = lo + share < n ? lo + share : n;
        part[i] = (ReadPart){ fd, buf + lo, off + (int64_t)lo, hi - lo, 0, 0 };
        if (i > 0 && part[i].n > 0) started[i] = pthread_create(&th[i], NULL, read_part, &part[i]) == 0;
    }
    read_part(&part[0]);
    for (int i = 1; i < np; i++) {
        if (started[i]) pthread_join(th[i], NULL);
        else read_part(&part[i]);   /* no thread: read it here */
    }
    for (int i = 0; i < np; i++) {
        if (part[i].err) {
            LOG("%s: read %s at %lld: %s", op, path, (long long)(part[i].off + (int64_t)part[i].got),
                part[i].err > 0 ? strerror(part[i].err) : "unexpected end of file");
            return 0;
        }
    }
    return 1;
}

/* [off, off + n) of file fd to device dst, in chunks through the two
 * staging buffers. */
static int stage_range(Stager *s, int fd, int64_t off, int64_t n, uint8_t *dst, const char *path, const char *op) {
    while (n > 0) {
        const size_t chunk = (size_t)(n < (int64_t)STAGE_BYTES ? n : (int64_t)STAGE_BYTES);
        const int k = s->k;
        hipError_t e = hipSuccess;
        if (s->used[k]) e = hipEventSynchronize(s->done[k]);   /* its previous copy has left the buffer */
        if (e != hipSuccess) {
            LOG("%s: copy to device: %s", op, hipGetErrorString(e));
            return 0;
        }
        if (!read_chunk(fd, (uint8_t *)s->host[k], off, chunk, path, op)) return 0;
        e = hipMemcpyAsync(dst, s->host[k], chunk, hipMemcpyHostToDevice, sepia_stream());
        if (e == hipSuccess) e = hipEventRecord(s->done[k], sepia_stream());
        if (e != hipSuccess) {
            LOG("%s: copy to device: %s", op, hipGetErrorString(e));
            return 0;
        }
        s->used[k] = 1;
        s->k ^= 1;
        off += (int64_t)chunk;
        dst += chunk;
        n -= (int64_t)chunk;
    }
    return 1;
}

/* ------------------------------------------------------ the manifest ---- */
struct SepiaResidentTable {
    SepiaResidentTensor *t;
    size_t n;
    char *bin_path;
    int64_t bin_size;
};

void sepia_hip_manifest_free(SepiaResidentTable *t) {
    if (!t) return;
    for (size_t i = 0; i < t->n; i++) free((char *)t->t[i].name);
    free(t->t);
    free(t->bin_path);
    free(t);
}

SepiaResidentTable *sepia_hip_manifest_load(const char *manifest_path, const char *resident_bin_path) {
    const char *op = "manifest_load";
    if (!manifest_path || !resident_bin_path) {
        LOG("%s: NULL path", op);
        return NULL;
    }
    int64_t bin_size;
    if (!file_size(resident_bin_path, &bin_size, op)) return NULL;
    SjValue *root = read_json(manifest_path, op);
    if (!root) return NULL;
    SepiaResidentTable *rt = (SepiaResidentTable *)calloc(1, sizeof *rt);
    const SjValue *tensors = sj_get(root, "tensors");
    if (!rt) {
        LOG("%s: out of host memory", op);
        goto fail;
    }
    if (!tensors || tensors->type != SJ_ARR) {
        LOG("%s: %s: missing 'tensors' array", op, manifest_path);
        goto fail;
    }
    rt->bin_size = bin_size;
    rt->bin_path = strdup(resident_bin_path);
    rt->t = (SepiaResidentTensor *)calloc(tensors->n ? tensors->n : 1, sizeof(SepiaResidentTensor));
    if (!rt->bin_path || !rt->t) {
        LOG("%s: out of host memory", op);
        goto fail;
    }
    for (size_t i = 0; i < tensors->n; i++) {
        const SjValue *jt = tensors->items[i];
        SepiaResidentTensor *e = &rt->t[i];
        const char *name = req_str(jt, "name", manifest_path, op);
        int64_t type;
        if (!name || !req_i64(jt, "ggml_type", &type, manifest_path, op) ||
            !req_i64(jt, "offset", &e->offset, manifest_path, op) ||
            !req_i64(jt, "nbytes", &e->nbytes, manifest_path, op))
            goto fail;
        e->name = strdup(name);
        if (!e->name) {
            LOG("%s: out of host memory", op);
            goto fail;
        }
        rt->n = i + 1;
        e->ggml_type = (int)type;
        const SjValue *shape = sj_get(jt, "shape");
        if (!shape || shape->type != SJ_ARR || shape->n == 0 || shape->n > 4) {
            LOG("%s: tensor '%s' has a missing/invalid 'shape' (1-4 dims expected)", op, e->name);
            goto fail;
        }
        e->n_dims = (int)shape->n;
        for (size_t d = 0; d < shape->n; d++) {
            const SjValue *v = shape->items[d];
            if (v->type != SJ_NUM || !v->is_int || v->i < 0) {
                LOG("%s: tensor '%s' has a non-integer dimension", op, e->name);
                goto fail;
            }
            e->shape[d] = v->i;
        }
        if (e->offset < 0 || e->nbytes < 0 || e->offset > bin_size || e->nbytes > bin_size - e->offset) {
            LOG("%s: tensor '%s' [%lld,%lld) exceeds resident.bin size %lld bytes", op, e->name,
                (long long)e->offset, (long long)(e->offset + e->nbytes), (long long)bin_size);
            goto fail;
        }
    }
    rt->n = tensors->n;
    sj_free(root);
    return rt;
fail:
    sj_free(root);
    sepia_hip_manifest_free(rt);
    return NULL;
}

size_t sepia_hip_manifest_count(const SepiaResidentTable *t) { return t ? t->n : 0; }

const SepiaResidentTensor *sepia_hip_manifest_tensor(const SepiaResidentTable *t, size_t i) {
    return (t && i < t->n) ? &t->t[i] : NULL;
}

const SepiaResidentTensor *sepia_hip_manifest_find(const SepiaResidentTable *t, const char *name) {
    if (!t || !name) return NULL;
    for (size_t i = 0; i < t->n; i++)
        if (strcmp(t->t[i].name, name) == 0) return &t->t[i];
    return NULL;
}

SepiaGpuBuf *sepia_hip_manifest_upload(const SepiaResidentTable *t) {
    const char *op = "manifest_upload";
    if (!t) {
        LOG("%s: NULL table", op);
        return NULL;
    }
    if (!sepia_ready(op)) return NULL;
    int64_t size;
    if (!file_size(t->bin_path, &size, op)) return NULL;
    if (size != t->bin_size) {
        LOG("%s: %s changed size since the manifest was loaded (%lld -> %lld bytes)", op, t->bin_path,
            (long long)t->bin_size, (long long)size);
        return NULL;
    }
    SepiaGpuBuf *buf = sepia_gpu_alloc(size > 0 ? (size_t)size : 1, 1);
    if (!buf) return NULL;
    const int fd = open(t->bin_path, O_RDONLY);
    if (fd < 0) {
        LOG("%s: open %s: %s", op, t->bin_path, strerror(errno));
        sepia_gpu_free(buf);
        return NULL;
    }
    Stager *s = stager_acquire(op);
    int ok = s && stage_range(s, fd, 0, size, sepia_buf_dev(buf), t->bin_path, op);
    if (s) stager_release(s);
    close(fd);
    if (ok && hipStreamSynchronize(sepia_stream()) != hipSuccess) {
        LOG("%s: stream error after the upload", op);
        ok = 0;
    }
    if (!ok) {
        sepia_gpu_free(buf);
        return NULL;
    }
    return buf;
}

/* ---------------------------------------------------- the expert index -- */
typedef struct {
    SepiaExpertSlot *slot[3];   /* [n_experts] each; NULL: no such layer */
} LayerSlots;

struct SepiaExpertIndex {
    char *index_path;
    char **parts;
    int n_parts;
    int n_experts;
    LayerSlots *layers;
    int n_layers;               /* entries in layers (max layer + 1) */
};

void sepia_hip_index_free(SepiaExpertIndex *idx) {
    if (!idx) return;
    for (int i = 0; i < idx->n_parts; i++) free(idx->parts[i]);
    free(idx->parts);
    for (int l = 0; l < idx->n_layers; l++)
        for (int k = 0; k < 3; k++) free(idx->layers[l].slot[k]);
    free(idx->layers);
    free(idx->index_path);
    free(idx);
}

static const char *const k_kinds[3] = { "gate", "up", "down" };

/* A layer key: decimal digits only. */
static int layer_key(const char *s) {
    if (!*s || strlen(s) > 6) return -1;
    int v = 0;
    for (const char *p = s; *p; p++) {
        if (*p < '0' || *p > '9') return -1;
        v = 10 * v + (*p - '0');
    }
    return v;
}

SepiaExpertIndex *sepia_hip_index_load(const char *index_path) {
    const char *op = "index_load";
    if (!index_path) {
        LOG("%s: NULL path", op);
        return NULL;
    }
    SjValue *root = read_json(index_path, op);
    if (!root) return NULL;
    SepiaExpertIndex *idx = (SepiaExpertIndex *)calloc(1, sizeof *idx);
    if (!idx || !(idx->index_path = strdup(index_path))) {
        LOG("%s: out of host memory", op);
        goto fail;
    }
    int64_t ne;
    if (!req_i64(root, "n_experts_per_layer", &ne, index_path, op)) goto fail;
    if (ne <= 0 || ne > (1 << 20)) {
        LOG("%s: n_experts_per_layer must be positive, got %lld", op, (long long)ne);
        goto fail;
    }
    idx->n_experts = (int)ne;
    const SjValue *parts = sj_get(root, "parts");
    if (!parts || parts->type != SJ_ARR) {
        LOG("%s: %s: missing 'parts' array", op, index_path);
        goto fail;
    }
    if (parts->n == 0 || parts->n > MAX_PARTS) {
        LOG("%s: 'parts' has %zu entries, expected 1-%d", op, parts->n, MAX_PARTS);
        goto fail;
    }
    idx->parts = (char **)calloc(parts->n, sizeof(char *));
    if (!idx->parts) goto oom;
    for (size_t i = 0; i < parts->n; i++) {
        const char *pf = req_str(parts->items[i], "part_file", index_path, op);
        if (!pf) goto fail;
        if (!(idx->parts[i] = strdup(pf))) goto oom;
        idx->n_parts = (int)i + 1;
    }
    const SjValue *moe = sj_get(root, "moe_layers");
    if (!moe || moe->type != SJ_OBJ) {
        LOG("%s: %s: missing 'moe_layers' object", op, index_path);
        goto fail;
    }
    int max_layer = -1;
    for (size_t i = 0; i < moe->n; i++) {
        const int l = layer_key(moe->keys[i]);
        if (l < 0) {
            LOG("%s: bad moe_layers key '%s'", op, moe->keys[i]);
            goto fail;
        }
        if (l > max_layer) max_layer = l;
    }
    idx->n_layers = max_layer + 1;
    idx->layers = (LayerSlots *)calloc(idx->n_layers > 0 ? (size_t)idx->n_layers : 1, sizeof(LayerSlots));
    if (!idx->layers) goto oom;
    for (size_t i = 0; i < moe->n; i++) {
        const int l = layer_key(moe->keys[i]);
        const SjValue *kinds = moe->items[i];
        if (idx->layers[l].slot[0]) {
            LOG("%s: layer %d appears twice", op, l);
            goto fail;
        }
        const SjValue *ko[3];
        for (int k = 0; k < 3; k++) ko[k] = sj_get(kinds, k_kinds[k]);
        if (!ko[0] || !ko[1] || !ko[2]) {
            LOG("%s: layer %d is missing gate/up/down (found gate=%d up=%d down=%d)", op, l, ko[0] != NULL,
                ko[1] != NULL, ko[2] != NULL);
            goto fail;
        }
        for (int k = 0; k < 3; k++) {
            const SjValue *ex = sj_get(ko[k], "experts");
            if (!ex || ex->type != SJ_ARR) {
                LOG("%s: layer %d slot '%s' missing 'experts' array", op, l, k_kinds[k]);
                goto fail;
            }
            if ((int64_t)ex->n != ne) {
                LOG("%s: layer %d slot '%s' has %zu experts, expected n_experts_per_layer=%d", op, l, k_kinds[k],
                    ex->n, idx->n_experts);
                goto fail;
            }
            SepiaExpertSlot *sl = (SepiaExpertSlot *)calloc(ex->n, sizeof(SepiaExpertSlot));
            if (!sl) goto oom;
            idx->layers[l].slot[k] = sl;
            for (size_t e = 0; e < ex->n; e++) {
                const SjValue *ent = ex->items[e];
                const char *pf = req_str(ent, "part_file", index_path, op);
                int64_t type;
                if (!pf || !req_i64(ent, "abs_offset", &sl[e].abs_offset, index_path, op) ||
                    !req_i64(ent, "nbytes", &sl[e].nbytes, index_path, op) ||
                    !req_i64(ent, "ggml_type", &type, index_path, op))
                    goto fail;
                sl[e].ggml_type = (int)type;
                sl[e].part_idx = -1;
                for (int p = 0; p < idx->n_parts; p++)
                    if (strcmp(idx->parts[p], pf) == 0) {
                        sl[e].part_idx = p;
                        break;
                    }
                if (sl[e].part_idx < 0) {
                    LOG("%s: layer %d slot '%s' expert %zu references unknown part_file '%s'", op, l, k_kinds[k], e,
                        pf);
                    goto fail;
                }
                if (sl[e].abs_offset < 0 || sl[e].nbytes < 0) {
                    LOG("%s: layer %d slot '%s' expert %zu has a negative offset/nbytes", op, l, k_kinds[k], e);
                    goto fail;
                }
            }
        }
    }
    sj_free(root);
    return idx;
oom:
    LOG("%s: out of host memory", op);
fail:
    sj_free(root);
    sepia_hip_index_free(idx);
    return NULL;
}

int sepia_hip_index_n_experts(const SepiaExpertIndex *idx) { return idx ? idx->n_experts : 0; }
int sepia_hip_index_n_parts(const SepiaExpertIndex *idx) { return idx ? idx->n_parts : 0; }
const char *sepia_hip_index_part(const SepiaExpertIndex *idx, int i) {
    return (idx && i >= 0 && i < idx->n_parts) ? idx->parts[i] : NULL;
}
int sepia_hip_index_has_layer(const SepiaExpertIndex *idx, int layer) {
    return idx && layer >= 0 && layer < idx->n_layers && idx->layers[layer].slot[0] != NULL;
}
int sepia_hip_index_slot(const SepiaExpertIndex *idx, int layer, int kind, int expert, SepiaExpertSlot *out) {
    if (!sepia_hip_index_has_layer(idx, layer) || kind < 0 || kind > 2 || expert < 0 || expert >= idx->n_experts ||
        !out)
        return 0;
    *out = idx->layers[layer].slot[kind][expert];
    return 1;
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

SepiaGpuBuf *sepia_hip_index_upload_layer(const SepiaExpertIndex *idx, const char *gguf_dir, int layer,
                                          SepiaExpertTensor out[3]) {
    const char *op = "index_upload_layer";
    if (!idx || !out) {
        LOG("%s: NULL argument", op);
        return NULL;
    }
    if (!sepia_hip_index_has_layer(idx, layer)) {
        LOG("%s: layer %d is not in the index", op, layer);
        return NULL;
    }
    if (!sepia_ready(op)) return NULL;
    const int ne = idx->n_experts;
    const LayerSlots *ls = &idx->layers[layer];
    size_t koff[3], total = 0;
    for (int k = 0; k < 3; k++) {
        const SepiaExpertSlot *sl = ls->slot[k];
        for (int e = 1; e < ne; e++)
            if (sl[e].ggml_type != sl[0].ggml_type || sl[e].nbytes != sl[0].nbytes) {
                LOG("%s: layer %d slot '%s': expert %d's type/size differs from expert 0's", op, layer, k_kinds[k], e);
                return NULL;
            }
        if (sl[0].nbytes <= 0) {
            LOG("%s: layer %d slot '%s' has empty experts", op, layer, k_kinds[k]);
            return NULL;
        }
        koff[k] = total;
        total = align_up(total + (size_t)ne * (size_t)sl[0].nbytes, 256);
    }
    char *dir = gguf_dir ? strdup(gguf_dir) : sibling(idx->index_path, "inkling-gguf");
    if (!dir) {
        LOG("%s: out of host memory", op);
        return NULL;
    }
    int fds[MAX_PARTS];
    int64_t sizes[MAX_PARTS];
    char *paths[MAX_PARTS];
    for (int p = 0; p < idx->n_parts; p++) {
        fds[p] = -1;
        paths[p] = NULL;
    }
    SepiaGpuBuf *buf = NULL;
    Stager *s = NULL;
    int ok = 0;
    for (int p = 0; p < idx->n_parts; p++) {
        paths[p] = (char *)malloc(strlen(dir) + strlen(idx->parts[p]) + 2);
        if (!paths[p]) {
            LOG("%s: out of host memory", op);
            goto done;
        }
        sprintf(paths[p], "%s/%s", dir, idx->parts[p]);
    }
    /* every slice inside its part, before anything is allocated */
    for (int k = 0; k < 3; k++)
        for (int e = 0; e < ne; e++) {
            const SepiaExpertSlot *sl = &ls->slot[k][e];
            const int p = sl->part_idx;
            if (fds[p] < 0) {
                if (!file_size(paths[p], &sizes[p], op)) goto done;
                fds[p] = open(paths[p], O_RDONLY);
                if (fds[p] < 0) {
                    LOG("%s: open %s: %s", op, paths[p], strerror(errno));
                    goto done;
                }
            }
            if (sl->abs_offset > sizes[p] || sl->nbytes > sizes[p] - sl->abs_offset) {
                LOG("%s: layer %d slot '%s' expert %d [%lld,+%lld) exceeds %s (%lld bytes)", op, layer, k_kinds[k], e,
                    (long long)sl->abs_offset, (long long)sl->nbytes, paths[p], (long long)sizes[p]);
                goto done;
            }
        }
    buf = sepia_gpu_alloc(total, 1);
    if (!buf) goto done;
    s = stager_acquire(op);
    if (!s) goto done;
    uint8_t *base = sepia_buf_dev(buf);
    for (int k = 0; k < 3; k++) {
        const SepiaExpertSlot *sl = ls->slot[k];
        const int64_t nb = sl[0].nbytes;
        for (int e = 0; e < ne;) {
            /* a run of experts back to back in one part reads as one range */
            int r = e + 1;
            while (r < ne && sl[r].part_idx == sl[e].part_idx && sl[r].abs_offset == sl[r - 1].abs_offset + nb) r++;
            if (!stage_range(s, fds[sl[e].part_idx], sl[e].abs_offset, (int64_t)(r - e) * nb,
                             base + koff[k] + (size_t)e * (size_t)nb, paths[sl[e].part_idx], op))
                goto done;
            e = r;
        }
        out[k].buf = buf;
        out[k].off = koff[k];
        out[k].stride = (size_t)nb;
        out[k].ggml_type = sl[0].ggml_type;
    }
    ok = 1;
done:
    if (s) stager_release(s);
    if (ok && hipStreamSynchronize(sepia_stream()) != hipSuccess) {
        LOG("%s: stream error after the upload", op);
        ok = 0;
    }
    for (int p = 0; p < idx->n_parts; p++) {
        if (fds[p] >= 0) close(fds[p]);
        free(paths[p]);
    }
    free(dir);
    if (!ok) {
        sepia_gpu_free(buf);
        return NULL;
    }
    return buf;
}

/* ------------------------------------------------ a layer from the stores */
static const SepiaResidentTensor *layer_tensor(const SepiaResidentTable *t, int layer, const char *suffix) {
    char name[160];
    const int n = snprintf(name, sizeof name, "blk.%d.%s", layer, suffix);
    if (n < 0 || (size_t)n >= sizeof name) return NULL;
    return sepia_hip_manifest_find(t, name);
}

/* An f32 tensor of numel elements. */
static int f32_tensor(const SepiaResidentTensor *e, int64_t numel, const char *op) {
    if (e->ggml_type != 0) {
        LOG("%s: resident tensor '%s': expected F32, got ggml_type %d", op, e->name, e->ggml_type);
        return 0;
    }
    int64_t n = 1;
    for (int d = 0; d < e->n_dims; d++) n *= e->shape[d];
    if (n != numel || e->nbytes != 4 * numel) {
        LOG("%s: resident tensor '%s': %lld elements / %lld bytes, expected %lld elements", op, e->name, (long long)n,
            (long long)e->nbytes, (long long)numel);
        return 0;
    }
    return 1;
}

/* A [rows, cols] matrix of type: stride bytes must hold it exactly. */
static int matrix_ok(int type, int64_t rows, int64_t cols, int64_t stride, const char *what, const char *op) {
    const int64_t rb = sepia_row_bytes(type, cols);
    if (rb < 0 || rb * rows != stride) {
        LOG("%s: %s: %lld bytes per matrix, expected %lld rows x %lld columns of ggml type %d", op, what,
            (long long)stride, (long long)rows, (long long)cols, type);
        return 0;
    }
    return 1;
}

int sepia_hip_moe_layer_from_stores(const SepiaResidentTable *t, SepiaGpuBuf *resident, int layer,
                                    const SepiaExpertTensor experts[3], int n_routed, int topk, float route_scale,
                                    SepiaMoeLayerDesc *out) {
    const char *op = "moe_layer_from_stores";
    if (!t || !resident || !experts || !out || n_routed < 1 || topk < 1 || topk > n_routed) {
        LOG("%s: invalid arguments", op);
        return 0;
    }
    if ((int64_t)sepia_buf_len(resident) < t->bin_size) {
        LOG("%s: the resident buffer is smaller than resident.bin", op);
        return 0;
    }
    const SepiaResidentTensor *rw = layer_tensor(t, layer, "ffn_gate_inp.weight");
    const SepiaResidentTensor *rb = layer_tensor(t, layer, "exp_probs_b.bias");
    const SepiaResidentTensor *gs = layer_tensor(t, layer, "ffn_gscale.weight");
    if (!rw || !rb || !gs) {
        LOG("%s: layer %d: resident router, bias or ffn_gscale tensor missing", op, layer);
        return 0;
    }
    if (rw->n_dims != 2 || rw->shape[1] < n_routed) {
        LOG("%s: '%s' must be [hidden, n_routed + n_shared]", op, rw->name);
        return 0;
    }
    const int64_t H = rw->shape[0];
    const int n_shared = (int)(rw->shape[1] - n_routed);
    if (!f32_tensor(rw, H * rw->shape[1], op) || !f32_tensor(rb, n_routed, op) || !f32_tensor(gs, 1, op)) return 0;
    float gscale;
    {
        const int fd = open(t->bin_path, O_RDONLY);
        const ssize_t r = fd >= 0 ? pread(fd, &gscale, 4, (off_t)gs->offset) : -1;
        if (fd >= 0) close(fd);
        if (r != 4) {
            LOG("%s: reading '%s' from %s failed", op, gs->name, t->bin_path);
            return 0;
        }
    }
    SepiaMoeLayerDesc d;
    memset(&d, 0, sizeof d);
    const SepiaResidentTensor *sh[3] = { NULL, NULL, NULL };
    int64_t I = -1;
    if (n_shared > 0) {
        static const char *const sfx[3] = { "ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight" };
        for (int k = 0; k < 3; k++) {
            sh[k] = layer_tensor(t, layer, sfx[k]);
            if (!sh[k] || sh[k]->n_dims != 3 || sh[k]->shape[2] != n_shared || sh[k]->nbytes % n_shared) {
                LOG("%s: layer %d: '%s' missing or not a stack of %d matrices", op, layer, sfx[k], n_shared);
                return 0;
            }
        }
        I = sh[0]->shape[1];
        const int64_t stride[3] = { sh[0]->nbytes / n_shared, sh[1]->nbytes / n_shared, sh[2]->nbytes / n_shared };
        if (sh[0]->shape[0] != H || sh[1]->shape[0] != H || sh[1]->shape[1] != I || sh[2]->shape[0] != I ||
            sh[2]->shape[1] != H || !matrix_ok(sh[0]->ggml_type, I, H, stride[0], sh[0]->name, op) ||
            !matrix_ok(sh[1]->ggml_type, I, H, stride[1], sh[1]->name, op) ||
            !matrix_ok(sh[2]->ggml_type, H, I, stride[2], sh[2]->name, op))
            return 0;
        SepiaExpertTensor *dst[3] = { &d.s_gate, &d.s_up, &d.s_down };
        for (int k = 0; k < 3; k++) {
            dst[k]->buf = resident;
            dst[k]->off = (size_t)sh[k]->offset;
            dst[k]->stride = (size_t)stride[k];
            dst[k]->ggml_type = sh[k]->ggml_type;
        }
    }
    /* the routed experts' inter from the gate stride when there is no shared expert */
    if (I < 0) {
        const int64_t rbg = sepia_row_bytes(experts[0].ggml_type, H);
        if (rbg <= 0 || (int64_t)experts[0].stride % rbg) {
            LOG("%s: routed gate stride %zu is not a whole number of rows of %lld columns", op, experts[0].stride,
                (long long)H);
            return 0;
        }
        I = (int64_t)experts[0].stride / rbg;
    }
    if (!matrix_ok(experts[0].ggml_type, I, H, (int64_t)experts[0].stride, "routed gate", op) ||
        !matrix_ok(experts[1].ggml_type, I, H, (int64_t)experts[1].stride, "routed up", op) ||
        !matrix_ok(experts[2].ggml_type, H, I, (int64_t)experts[2].stride, "routed down", op))
        return 0;
    d.hidden = H;
    d.inter = I;
    d.n_routed = n_routed;
    d.n_shared = n_shared;
    d.topk = topk;
    d.route_scale = route_scale;
    d.global_scale = gscale;
    d.router_w = resident;
    d.router_w_off = (size_t)rw->offset;
    d.router_bias = resident;
    d.router_bias_off = (size_t)rb->offset;
    d.gate = experts[0];
    d.up = experts[1];
    d.down = experts[2];
    *out = d;
    return 1;
}
