/* s2pro MI355X — prequantized-weight sidecar cache (include/s2pro/qcache.h).
 *
 * On-disk layout, kept byte-compatible with the reference
 * (src/sched/qcache.c:1-16; little-endian, payload offsets absolute and
 * 256-aligned, payloads in entry order, zero padding between them):
 *   u8 magic[8] "S2PQC\1\0\0" | u64 fingerprint | u32 n_entries | u32 0
 *   n x { u32 name_len, u32 kind, i32 N, i32 K, i32 group, u32 0,
 *         u64 q_off, u64 q_len, u64 s_off, u64 s_len, char name[name_len] }
 *   payloads
 * kind 1: per-channel INT8 (i8 [N][K], f32 [N]); kind 2: packed INT4
 * (u8 [N][K/2], f16 [N][K/G]); kind 3: INT4 codes in int8 (i8 [N][K],
 * f16 [N][K/G]).
 *
 * Reading maps the file instead of copying it into memory: the header is
 * parsed and bounds-checked in place, and a hit uploads straight from the
 * mapping; the mapping is released by s2p_qcache_finish once the stream's
 * uploads are complete.  Writing snapshots each linear's device tensors to
 * host memory at put time and writes the file at finish through a temporary
 * file and a rename, so a reader never sees a partial cache.  Every read
 * failure degrades to a miss and every write failure to "no cache". */
#define _GNU_SOURCE
#include "s2pro/qcache.h"

#include <dirent.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#define QC_HDR 24
#define QC_ENT 56
#define QC_ALIGN 256
#define QC_MAX 512
#define QC_MAX_NAME 512
#define QC_MAX_FILES 256

static const unsigned char qc_magic[8] = {'S', '2', 'P', 'Q', 'C', 1, 0, 0};

typedef struct {
    char* name;
    uint32_t kind;
    int32_t N, K, group;
    uint64_t q_off, q_len, s_off, s_len;
    void* qh; /* write mode: host snapshots */
    void* sh;
} qc_ent;

struct s2p_qcache {
    char path[1024];
    int reading;
    uint64_t fp;
    unsigned char* map; /* read mode: the mapped file */
    size_t map_len;
    int n;
    qc_ent e[QC_MAX];
};

/* FNV-1a, 64-bit (offset basis 0xcbf29ce484222325, prime 0x100000001b3) */
static uint64_t fnv1a(uint64_t h, const void* p, size_t n) {
    const unsigned char* b = (const unsigned char*)p;
    for (size_t i = 0; i < n; i++) h = (h ^ b[i]) * 0x100000001b3ull;
    return h;
}

/* unset or empty: def; exactly "1": 1; anything else: 0 */
static int env_flag(const char* name, int def) {
    const char* v = getenv(name);
    if (!v || !v[0]) return def;
    return strcmp(v, "1") == 0;
}

static int by_name(const void* a, const void* b) {
    return strcmp(*(char* const*)a, *(char* const*)b);
}

/* the quantisation config string, then (name, size, mtime) of every
 * *.safetensors of the directory in name order */
static int fingerprint(const char* dir, s2p_gemm_mode mode, uint64_t* out) {
    char cfg[256];
    const char* g = getenv("S2P_INT4_GROUP");
    snprintf(cfg, sizeof(cfg), "v1|mode=%d|int4=%d|g=%s|mse=%d|pk=%d|all=%d", (int)mode,
             env_flag("S2P_INT4", 0), g ? g : "32", env_flag("S2P_INT4_MSE", 1),
             env_flag("S2P_INT4_PACKED", 1), env_flag("S2P_INT4_ALL", 0));
    uint64_t h = fnv1a(0xcbf29ce484222325ull, cfg, strlen(cfg));
    DIR* d = opendir(dir);
    if (!d) return -1;
    char* names[QC_MAX_FILES];
    int n = 0;
    for (struct dirent* de; (de = readdir(d)) != NULL && n < QC_MAX_FILES;) {
        const size_t len = strlen(de->d_name);
        if (len > 12 && strcmp(de->d_name + len - 12, ".safetensors") == 0) {
            names[n] = strdup(de->d_name);
            if (names[n]) n++;
        }
    }
    closedir(d);
    if (n == 0) return -1;
    qsort(names, (size_t)n, sizeof(names[0]), by_name);
    for (int i = 0; i < n; i++) {
        char full[1400];
        struct stat st;
        snprintf(full, sizeof(full), "%s/%s", dir, names[i]);
        if (stat(full, &st) == 0) {
            const int64_t size = (int64_t)st.st_size, mtime = (int64_t)st.st_mtime;
            h = fnv1a(h, names[i], strlen(names[i]));
            h = fnv1a(h, &size, 8);
            h = fnv1a(h, &mtime, 8);
        }
        free(names[i]);
    }
    *out = h;
    return 0;
}

static uint32_t rd32(const unsigned char* p) {
    uint32_t v;
    memcpy(&v, p, 4);
    return v;
}
static uint64_t rd64(const unsigned char* p) {
    uint64_t v;
    memcpy(&v, p, 8);
    return v;
}
/* [off, off + len) inside a file of sz bytes, without overflow */
static int in_file(uint64_t off, uint64_t len, uint64_t sz) { return off <= sz && len <= sz - off; }

static void drop_entries(s2p_qcache* qc) {
    for (int i = 0; i < qc->n; i++) {
        free(qc->e[i].name);
        free(qc->e[i].qh);
        free(qc->e[i].sh);
    }
    memset(qc->e, 0, sizeof(qc->e[0]) * (size_t)qc->n);
    qc->n = 0;
}

/* map the file and parse its header; any inconsistency leaves write mode */
static void read_header(s2p_qcache* qc) {
    const int fd = open(qc->path, O_RDONLY);
    if (fd < 0) return;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < QC_HDR) {
        close(fd);
        return;
    }
    const uint64_t sz = (uint64_t)st.st_size;
    unsigned char* m = (unsigned char*)mmap(NULL, (size_t)sz, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return;
    const uint32_t n = rd32(m + 16);
    int ok = memcmp(m, qc_magic, 8) == 0 && n > 0 && n <= QC_MAX;
    if (ok && rd64(m + 8) != qc->fp) {
        fprintf(stderr, "[s2pro] qcache: stale fingerprint, rebuilding\n");
        ok = 0;
    }
    uint64_t off = QC_HDR;
    for (uint32_t i = 0; ok && i < n; i++) {
        if (!in_file(off, QC_ENT, sz)) {
            ok = 0;
            break;
        }
        const unsigned char* h = m + off;
        qc_ent* e = &qc->e[i];
        const uint32_t name_len = rd32(h);
        e->kind = rd32(h + 4);
        memcpy(&e->N, h + 8, 4);
        memcpy(&e->K, h + 12, 4);
        memcpy(&e->group, h + 16, 4);
        e->q_off = rd64(h + 24);
        e->q_len = rd64(h + 32);
        e->s_off = rd64(h + 40);
        e->s_len = rd64(h + 48);
        off += QC_ENT;
        if (name_len == 0 || name_len > QC_MAX_NAME || !in_file(off, name_len, sz) ||
            !in_file(e->q_off, e->q_len, sz) || !in_file(e->s_off, e->s_len, sz) ||
            !(e->name = (char*)malloc(name_len + 1))) {
            ok = 0;
            break;
        }
        memcpy(e->name, m + off, name_len);
        e->name[name_len] = '\0';
        off += name_len;
        qc->n = (int)i + 1;
    }
    if (!ok) {
        drop_entries(qc);
        munmap(m, (size_t)sz);
        return;
    }
    qc->map = m;
    qc->map_len = (size_t)sz;
    qc->reading = 1;
}

s2p_status s2p_qcache_open(const char* model_dir, s2p_gemm_mode mode, s2p_qcache** out) {
    if (!model_dir || !out) return S2P_ERR_INVALID;
    *out = NULL;
    if (mode != S2P_GEMM_INT8 || !env_flag("S2P_QCACHE", 1)) return S2P_OK;
    s2p_qcache* qc = (s2p_qcache*)calloc(1, sizeof(*qc));
    if (!qc) return S2P_ERR_OOM;
    if (fingerprint(model_dir, mode, &qc->fp) != 0) { /* unusual model dir: no cache */
        free(qc);
        return S2P_OK;
    }
    const char* dir = getenv("S2P_QCACHE_DIR");
    snprintf(qc->path, sizeof(qc->path), "%s/s2p_qcache.bin", dir && dir[0] ? dir : model_dir);
    read_header(qc);
    if (qc->reading)
        fprintf(stderr, "[s2pro] qcache: serving %d tensors from %s\n", qc->n, qc->path);
    else
        fprintf(stderr, "[s2pro] qcache: will write %s after load\n", qc->path);
    *out = qc;
    return S2P_OK;
}

int s2p_qcache_reading(const s2p_qcache* qc) { return qc && qc->reading; }

/* the device tensors of an entry: codes (w_pack for kind 2, else w_int8)
 * and scales, with the reference's dtypes and shapes */
static s2p_status alloc_entry(const qc_ent* e, s2p_linear* lin, s2p_tensor** qt) {
    if (e->N <= 0 || e->K <= 0) return S2P_ERR_FORMAT;
    if (e->kind >= 2 && (e->group <= 0 || e->K % e->group)) return S2P_ERR_FORMAT;
    s2p_status rc;
    if (e->kind == 1) {
        const int64_t qs[2] = {e->N, e->K}, ss[1] = {e->N};
        *qt = &lin->w_int8;
        rc = s2p_tensor_device_alloc(&lin->w_int8, S2P_DT_I8, 2, qs);
        if (rc == S2P_OK) rc = s2p_tensor_device_alloc(&lin->w_iscale, S2P_DT_F32, 1, ss);
    } else if (e->kind == 2 || e->kind == 3) {
        const int64_t qs[2] = {e->N, e->kind == 2 ? e->K / 2 : e->K};
        const int64_t ss[1] = {(int64_t)e->N * (e->K / e->group)};
        *qt = e->kind == 2 ? &lin->w_pack : &lin->w_int8;
        rc = s2p_tensor_device_alloc(*qt, S2P_DT_I8, 2, qs);
        if (rc == S2P_OK) rc = s2p_tensor_device_alloc(&lin->w_iscale, S2P_DT_F16, 1, ss);
    } else {
        return S2P_ERR_FORMAT;
    }
    if (rc == S2P_OK && ((*qt)->bytes != e->q_len || lin->w_iscale.bytes != e->s_len))
        rc = S2P_ERR_FORMAT;
    return rc;
}

int s2p_qcache_try_load(s2p_qcache* qc, const char* name, int in_features, int out_features,
                        s2p_linear* lin, hipStream_t stream) {
    if (!qc || !qc->reading || !name || !lin) return 0;
    const qc_ent* e = NULL;
    for (int i = 0; i < qc->n && !e; i++)
        if (strcmp(qc->e[i].name, name) == 0) e = &qc->e[i];
    if (!e) {
        fprintf(stderr, "[s2pro] qcache: miss for %s (live path)\n", name);
        return 0;
    }
    if (e->N != out_features || e->K != in_features) {
        fprintf(stderr, "[s2pro] qcache: shape mismatch for %s\n", name);
        return 0;
    }
    memset(lin, 0, sizeof(*lin));
    lin->in_features = in_features;
    lin->out_features = out_features;
    s2p_tensor* qt = NULL;
    s2p_status rc = alloc_entry(e, lin, &qt);
    if (rc == S2P_ERR_FORMAT) fprintf(stderr, "[s2pro] qcache: size mismatch for %s\n", name);
    if (rc == S2P_OK &&
        (hipMemcpyAsync(qt->data, qc->map + e->q_off, e->q_len, hipMemcpyHostToDevice, stream) !=
             hipSuccess ||
         hipMemcpyAsync(lin->w_iscale.data, qc->map + e->s_off, e->s_len, hipMemcpyHostToDevice,
                        stream) != hipSuccess))
        rc = S2P_ERR_CUDA;
    if (rc != S2P_OK) {
        s2p_tensor_free(&lin->w_int8);
        s2p_tensor_free(&lin->w_pack);
        s2p_tensor_free(&lin->w_iscale);
        memset(lin, 0, sizeof(*lin));
        lin->in_features = in_features;
        lin->out_features = out_features;
        return 0;
    }
    lin->int8_ready = 1;
    if (e->kind >= 2) lin->q_group = e->group;
    if (e->kind == 2) lin->q_packed = 1;
    return 1;
}

s2p_status s2p_qcache_put_linear(s2p_qcache* qc, const char* name, const s2p_linear* lin,
                                 hipStream_t stream) {
    if (!qc || qc->reading || !name || !lin || !lin->int8_ready || qc->n >= QC_MAX) return S2P_OK;
    const s2p_tensor* qt = lin->q_packed ? &lin->w_pack : &lin->w_int8;
    if (!qt->data || !lin->w_iscale.data || strlen(name) == 0 || strlen(name) > QC_MAX_NAME)
        return S2P_OK;
    qc_ent* e = &qc->e[qc->n];
    memset(e, 0, sizeof(*e));
    e->kind = lin->q_packed ? 2u : (lin->q_group > 0 ? 3u : 1u);
    e->N = lin->out_features;
    e->K = lin->in_features;
    e->group = lin->q_group;
    e->q_len = qt->bytes;
    e->s_len = lin->w_iscale.bytes;
    e->name = strdup(name);
    e->qh = malloc(e->q_len ? e->q_len : 1);
    e->sh = malloc(e->s_len ? e->s_len : 1);
    if (!e->name || !e->qh || !e->sh) { /* the cache degrades, the load does not */
        free(e->name);
        free(e->qh);
        free(e->sh);
        memset(e, 0, sizeof(*e));
        return S2P_OK;
    }
    if (hipStreamSynchronize(stream) != hipSuccess ||
        hipMemcpy(e->qh, qt->data, e->q_len, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpy(e->sh, lin->w_iscale.data, e->s_len, hipMemcpyDeviceToHost) != hipSuccess) {
        free(e->name);
        free(e->qh);
        free(e->sh);
        memset(e, 0, sizeof(*e));
        return S2P_ERR_CUDA;
    }
    qc->n++;
    return S2P_OK;
}

static uint64_t align_up(uint64_t v) { return (v + QC_ALIGN - 1) & ~(uint64_t)(QC_ALIGN - 1); }

/* zeros up to byte offset to, then len bytes of p */
static int put_at(FILE* f, uint64_t* pos, uint64_t to, const void* p, uint64_t len) {
    static const unsigned char zeros[QC_ALIGN];
    while (*pos < to) {
        const size_t k = (size_t)(to - *pos < QC_ALIGN ? to - *pos : QC_ALIGN);
        if (fwrite(zeros, 1, k, f) != k) return 0;
        *pos += k;
    }
    if (len && fwrite(p, 1, (size_t)len, f) != (size_t)len) return 0;
    *pos += len;
    return 1;
}

static s2p_status write_file(s2p_qcache* qc) {
    /* header and entry table in one buffer; payload offsets after it */
    uint64_t table = QC_HDR;
    for (int i = 0; i < qc->n; i++) table += QC_ENT + strlen(qc->e[i].name);
    uint64_t off = table;
    for (int i = 0; i < qc->n; i++) {
        qc_ent* e = &qc->e[i];
        e->q_off = off = align_up(off);
        off += e->q_len;
        e->s_off = off = align_up(off);
        off += e->s_len;
    }
    unsigned char* hb = (unsigned char*)calloc(1, (size_t)table);
    if (!hb) return S2P_ERR_OOM;
    memcpy(hb, qc_magic, 8);
    memcpy(hb + 8, &qc->fp, 8);
    const uint32_t n32 = (uint32_t)qc->n;
    memcpy(hb + 16, &n32, 4);
    unsigned char* p = hb + QC_HDR;
    for (int i = 0; i < qc->n; i++) {
        const qc_ent* e = &qc->e[i];
        const uint32_t nl = (uint32_t)strlen(e->name);
        memcpy(p, &nl, 4);
        memcpy(p + 4, &e->kind, 4);
        memcpy(p + 8, &e->N, 4);
        memcpy(p + 12, &e->K, 4);
        memcpy(p + 16, &e->group, 4);
        memcpy(p + 24, &e->q_off, 8);
        memcpy(p + 32, &e->q_len, 8);
        memcpy(p + 40, &e->s_off, 8);
        memcpy(p + 48, &e->s_len, 8);
        memcpy(p + QC_ENT, e->name, nl);
        p += QC_ENT + nl;
    }
    char tmp[1100];
    snprintf(tmp, sizeof(tmp), "%s.tmp", qc->path);
    FILE* f = fopen(tmp, "wb");
    if (!f) {
        free(hb);
        fprintf(stderr, "[s2pro] qcache: cannot write %s (skipping)\n", tmp);
        return S2P_OK;
    }
    uint64_t pos = 0;
    int ok = put_at(f, &pos, 0, hb, table);
    free(hb);
    for (int i = 0; ok && i < qc->n; i++) {
        const qc_ent* e = &qc->e[i];
        ok = put_at(f, &pos, e->q_off, e->qh, e->q_len) && put_at(f, &pos, e->s_off, e->sh, e->s_len);
    }
    ok = (fclose(f) == 0) && ok;
    if (!ok || rename(tmp, qc->path) != 0) {
        fprintf(stderr, "[s2pro] qcache: write failed (%s), removing\n", tmp);
        remove(tmp);
        return S2P_OK;
    }
    fprintf(stderr, "[s2pro] qcache: wrote %d tensors -> %s\n", qc->n, qc->path);
    return S2P_OK;
}

s2p_status s2p_qcache_finish(s2p_qcache* qc, hipStream_t stream) {
    if (!qc) return S2P_OK;
    if (qc->reading) { /* uploads read the mapping: they must be complete */
        if (hipStreamSynchronize(stream) != hipSuccess) return S2P_ERR_CUDA;
        if (qc->map) munmap(qc->map, qc->map_len);
        qc->map = NULL;
        qc->map_len = 0;
        return S2P_OK;
    }
    return qc->n ? write_file(qc) : S2P_OK;
}

void s2p_qcache_free(s2p_qcache* qc) {
    if (!qc) return;
    drop_entries(qc);
    if (qc->map) munmap(qc->map, qc->map_len);
    free(qc);
}
