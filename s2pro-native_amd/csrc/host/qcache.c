/* s2pro MI355X — prequantized-weight sidecar cache (include/s2pro/qcache.h).
 *
 * File format (kept so that a file written by either build is read by the
 * other; reference src/sched/qcache.c:1-16): little-endian;
 *   [0,8)   magic "S2PQC" 1 0 0      [8,16)  u64 stamp of the weights/settings
 *   [16,20) u32 descriptor count     [20,24) u32 zero
 *   count descriptors of 56 bytes, each followed by its name (no NUL):
 *     u32 name bytes, u32 kind, i32 N, i32 K, i32 group, u32 zero,
 *     u64 codes offset, u64 codes bytes, u64 scales offset, u64 scales bytes
 *   payloads at absolute 256-aligned offsets, in descriptor order, codes then
 *   scales, zero padding between them.
 * Kinds: 1 per-channel INT8 (i8 [N][K] + f32 [N]), 2 packed INT4 (u8
 * [N][K/2] + f16 [N][K/group]), 3 INT4 codes one per byte (i8 [N][K] + f16
 * [N][K/group]).
 *
 * This implementation never holds a whole model on the host:
 * - Reading keeps the file open and only its descriptor table in memory
 *   (sorted by name for lookups).  A hit streams the payload with pread()
 *   through two pinned staging chunks, each H2D copy overlapping the next
 *   read; a chunk is reused once the event recorded after its copy has
 *   completed.  A file that shrinks or fails to read mid-load turns that
 *   lookup into a miss (no mapping, so no SIGBUS).
 * - Writing spools each linear's payload to a side file as it is put (one
 *   bounded host chunk at a time) and, at finish, writes header + table +
 *   the spooled payloads to a temporary file that is renamed over the cache,
 *   so readers never see a partial file.
 * Every read failure is a miss (the caller quantises live) and every write
 * failure leaves no cache behind. */
#define _GNU_SOURCE
#include "s2pro/qcache.h"

#include <dirent.h>
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

enum {
    HEAD_BYTES = 24,
    DESC_BYTES = 56,
    PAYLOAD_ALIGN = 256,
    MAX_DESCS = 512,
    MAX_NAME = 512,
    MAX_WEIGHT_FILES = 256,
};
#define CHUNK_BYTES ((size_t)8 << 20)

static const unsigned char k_magic[8] = {0x53, 0x32, 0x50, 0x51, 0x43, 0x01, 0x00, 0x00};

typedef struct {
    char* name;
    uint32_t kind;
    int32_t n, k, group;
    uint64_t codes_at, codes_len, scales_at, scales_len; /* write mode: spool-relative */
} qc_desc;

struct s2p_qcache {
    char file[1024];
    int reading;
    uint64_t stamp;
    int count;
    qc_desc desc[MAX_DESCS];
    /* read mode */
    int fd;
    uint64_t file_len;
    int by_name[MAX_DESCS];
    unsigned char* stage[2];
    int stage_pinned;
    hipEvent_t copied[2];
    int copied_live[2];
    int turn;
    /* write mode */
    FILE* spool;
    char spool_path[1100];
    uint64_t spool_len;
    int spool_failed;
};

/* ------------------------------------------------------------- helpers */

static uint64_t fnv1a64(uint64_t h, const void* bytes, size_t n) {
    for (const unsigned char *p = (const unsigned char*)bytes, *e = p + n; p < e; p++) {
        h ^= *p;
        h *= 0x100000001b3ull;
    }
    return h;
}

static uint32_t get_u32(const unsigned char* p) {
    return (uint32_t)p[0] | (uint32_t)p[1] << 8 | (uint32_t)p[2] << 16 | (uint32_t)p[3] << 24;
}
static uint64_t get_u64(const unsigned char* p) { return get_u32(p) | (uint64_t)get_u32(p + 4) << 32; }
static void put_u32(unsigned char* p, uint32_t v) {
    for (int i = 0; i < 4; i++) p[i] = (unsigned char)(v >> (8 * i));
}
static void put_u64(unsigned char* p, uint64_t v) {
    put_u32(p, (uint32_t)v);
    put_u32(p + 4, (uint32_t)(v >> 32));
}
static uint64_t round_up(uint64_t v) { return (v + PAYLOAD_ALIGN - 1) / PAYLOAD_ALIGN * PAYLOAD_ALIGN; }

/* a settings switch: unset or empty -> fallback, "1" -> 1, else 0 */
static int switch_on(const char* var, int fallback) {
    const char* v = getenv(var);
    return (!v || !*v) ? fallback : strcmp(v, "1") == 0;
}

typedef struct {
    char name[256];
    int64_t size, mtime;
} weight_file;

static int weight_file_order(const void* a, const void* b) {
    return strcmp(((const weight_file*)a)->name, ((const weight_file*)b)->name);
}

/* The stamp a cache file must carry to be served: FNV-1a 64 over the
 * quantisation settings string, then name, size and mtime of every
 * *.safetensors of the model directory in byte order of the names
 * (reference qcache.c:69-107; the string and the order are the format). */
static int weights_stamp(const char* dir, s2p_gemm_mode mode, uint64_t* stamp) {
    DIR* d = opendir(dir);
    if (!d) return -1;
    weight_file* files = (weight_file*)malloc(sizeof(weight_file) * MAX_WEIGHT_FILES);
    if (!files) {
        closedir(d);
        return -1;
    }
    int n = 0;
    const struct dirent* de;
    while (n < MAX_WEIGHT_FILES && (de = readdir(d)) != NULL) {
        const size_t len = strlen(de->d_name);
        if (len <= 12 || len >= sizeof(files[0].name) ||
            memcmp(de->d_name + len - 12, ".safetensors", 12) != 0)
            continue;
        char path[1400];
        struct stat st;
        snprintf(path, sizeof(path), "%s/%s", dir, de->d_name);
        if (stat(path, &st) != 0) continue;
        memcpy(files[n].name, de->d_name, len + 1);
        files[n].size = (int64_t)st.st_size;
        files[n].mtime = (int64_t)st.st_mtime;
        n++;
    }
    closedir(d);
    if (n == 0) {
        free(files);
        return -1;
    }
    qsort(files, (size_t)n, sizeof(files[0]), weight_file_order);
    const char* group = getenv("S2P_INT4_GROUP");
    char settings[256];
    const int sl = snprintf(settings, sizeof(settings), "v1|mode=%d|int4=%d|g=%s|mse=%d|pk=%d|all=%d",
                            (int)mode, switch_on("S2P_INT4", 0), group ? group : "32",
                            switch_on("S2P_INT4_MSE", 1), switch_on("S2P_INT4_PACKED", 1),
                            switch_on("S2P_INT4_ALL", 0));
    uint64_t h = fnv1a64(0xcbf29ce484222325ull, settings, (size_t)sl);
    for (int i = 0; i < n; i++) {
        h = fnv1a64(h, files[i].name, strlen(files[i].name));
        h = fnv1a64(h, &files[i].size, 8);
        h = fnv1a64(h, &files[i].mtime, 8);
    }
    free(files);
    *stamp = h;
    return 0;
}

/* payload bytes a descriptor of this kind and shape must have; 0: invalid */
static int expected_lengths(uint32_t kind, int32_t n, int32_t k, int32_t group, uint64_t* codes,
                            uint64_t* scales) {
    if (n <= 0 || k <= 0) return 0;
    const uint64_t N = (uint64_t)n, K = (uint64_t)k;
    switch (kind) {
    case 1:
        *codes = N * K;
        *scales = 4 * N;
        return 1;
    case 2:
    case 3:
        if (group <= 0 || k % group || (kind == 2 && k % 2)) return 0;
        *codes = kind == 2 ? N * K / 2 : N * K;
        *scales = 2 * N * (K / (uint64_t)group);
        return 1;
    default:
        return 0;
    }
}

static void forget_descs(s2p_qcache* qc) {
    for (int i = 0; i < qc->count; i++) free(qc->desc[i].name);
    qc->count = 0;
}

/* ---------------------------------------------------------------- read */

static int pread_all(int fd, void* dst, size_t len, uint64_t at) {
    unsigned char* p = (unsigned char*)dst;
    while (len) {
        const ssize_t got = pread(fd, p, len, (off_t)at);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return 0;
        p += got;
        len -= (size_t)got;
        at += (uint64_t)got;
    }
    return 1;
}

static int desc_order(const void* a, const void* b, void* ctx) {
    const s2p_qcache* qc = (const s2p_qcache*)ctx;
    const int i = *(const int*)a, j = *(const int*)b;
    const int c = strcmp(qc->desc[i].name, qc->desc[j].name);
    return c ? c : (i > j) - (i < j); /* equal names: table order, so the first one wins */
}

/* Parse header and table of an open cache file; 1 when it is servable. */
static int load_table(s2p_qcache* qc) {
    unsigned char head[HEAD_BYTES];
    if (qc->file_len < HEAD_BYTES || !pread_all(qc->fd, head, HEAD_BYTES, 0)) return 0;
    if (memcmp(head, k_magic, sizeof(k_magic)) != 0) return 0;
    const uint32_t count = get_u32(head + 16);
    if (count == 0 || count > MAX_DESCS) return 0;
    if (get_u64(head + 8) != qc->stamp) {
        fprintf(stderr, "[s2pro] qcache: %s was made for other weights or settings; "
                        "it will be regenerated\n", qc->file);
        return 0;
    }
    /* the table is at most count x (descriptor + longest name) */
    uint64_t span = (uint64_t)count * (DESC_BYTES + MAX_NAME);
    if (span > qc->file_len - HEAD_BYTES) span = qc->file_len - HEAD_BYTES;
    unsigned char* table = (unsigned char*)malloc((size_t)span + 1);
    if (!table) return 0;
    int ok = pread_all(qc->fd, table, (size_t)span, HEAD_BYTES);
    uint64_t at = 0;
    for (uint32_t i = 0; ok && i < count; i++) {
        if (span - at < DESC_BYTES) {
            ok = 0;
            break;
        }
        const unsigned char* r = table + at;
        const uint32_t name_len = get_u32(r);
        qc_desc d = {0};
        d.kind = get_u32(r + 4);
        d.n = (int32_t)get_u32(r + 8);
        d.k = (int32_t)get_u32(r + 12);
        d.group = (int32_t)get_u32(r + 16);
        d.codes_at = get_u64(r + 24);
        d.codes_len = get_u64(r + 32);
        d.scales_at = get_u64(r + 40);
        d.scales_len = get_u64(r + 48);
        at += DESC_BYTES;
        const uint64_t L = qc->file_len;
        ok = name_len >= 1 && name_len <= MAX_NAME && span - at >= name_len &&
             d.codes_at <= L && d.codes_len <= L - d.codes_at && d.scales_at <= L &&
             d.scales_len <= L - d.scales_at;
        if (ok) ok = (d.name = strndup((const char*)table + at, name_len)) != NULL;
        if (ok) {
            qc->desc[qc->count++] = d;
            at += name_len;
        }
    }
    free(table);
    if (!ok) {
        forget_descs(qc);
        return 0;
    }
    for (int i = 0; i < qc->count; i++) qc->by_name[i] = i;
    qsort_r(qc->by_name, (size_t)qc->count, sizeof(int), desc_order, qc);
    return 1;
}

static const qc_desc* lookup(const s2p_qcache* qc, const char* name) {
    int lo = 0, hi = qc->count; /* first entry whose name is >= name */
    while (lo < hi) {
        const int mid = (lo + hi) / 2;
        if (strcmp(qc->desc[qc->by_name[mid]].name, name) < 0) lo = mid + 1;
        else hi = mid;
    }
    if (lo < qc->count && strcmp(qc->desc[qc->by_name[lo]].name, name) == 0)
        return &qc->desc[qc->by_name[lo]];
    return NULL;
}

static int staging_ready(s2p_qcache* qc) {
    if (qc->stage[0]) return 1;
    if (hipHostMalloc((void**)&qc->stage[0], 2 * CHUNK_BYTES, hipHostMallocDefault) == hipSuccess) {
        qc->stage_pinned = 1;
    } else {
        (void)hipGetLastError();
        qc->stage[0] = (unsigned char*)malloc(2 * CHUNK_BYTES); /* synchronous copies then */
        if (!qc->stage[0]) return 0;
    }
    qc->stage[1] = qc->stage[0] + CHUNK_BYTES;
    return 1;
}

/* file bytes [at, at + len) -> device dst, through the staging chunks */
static int stream_payload(s2p_qcache* qc, uint64_t at, uint64_t len, void* dst, hipStream_t st) {
    if (!staging_ready(qc)) return 0;
    for (uint64_t done = 0; done < len;) {
        const size_t n = (size_t)(len - done < CHUNK_BYTES ? len - done : CHUNK_BYTES);
        const int c = qc->turn;
        qc->turn ^= 1;
        unsigned char* buf = qc->stage[c];
        if (qc->copied_live[c] && hipEventSynchronize(qc->copied[c]) != hipSuccess) return 0;
        if (!pread_all(qc->fd, buf, n, at + done)) return 0;
        void* d = (unsigned char*)dst + done;
        if (!qc->stage_pinned) {
            if (hipMemcpy(d, buf, n, hipMemcpyHostToDevice) != hipSuccess) return 0;
        } else {
            if (!qc->copied_live[c]) {
                if (hipEventCreateWithFlags(&qc->copied[c], hipEventDisableTiming) != hipSuccess)
                    return 0;
                qc->copied_live[c] = 1;
            }
            if (hipMemcpyAsync(d, buf, n, hipMemcpyHostToDevice, st) != hipSuccess ||
                hipEventRecord(qc->copied[c], st) != hipSuccess)
                return 0;
        }
        done += n;
    }
    return 1;
}

/* uploads still reading the staging chunks must finish before they go */
static int drain_staging(s2p_qcache* qc) {
    int ok = 1;
    for (int c = 0; c < 2; c++)
        if (qc->copied_live[c]) {
            ok = hipEventSynchronize(qc->copied[c]) == hipSuccess && ok;
            (void)hipEventDestroy(qc->copied[c]);
            qc->copied_live[c] = 0;
        }
    return ok;
}

static void release_reader(s2p_qcache* qc) {
    (void)drain_staging(qc);
    if (qc->stage[0]) {
        if (qc->stage_pinned) (void)hipHostFree(qc->stage[0]);
        else free(qc->stage[0]);
    }
    qc->stage[0] = qc->stage[1] = NULL;
    if (qc->fd >= 0) close(qc->fd);
    qc->fd = -1;
}

int s2p_qcache_try_load(s2p_qcache* qc, const char* name, int in_features, int out_features,
                        s2p_linear* lin, hipStream_t stream) {
    if (!qc || !qc->reading || qc->fd < 0 || !name || !lin) return 0;
    const qc_desc* d = lookup(qc, name);
    if (!d) {
        fprintf(stderr, "[s2pro] qcache: %s is not cached; quantising it live\n", name);
        return 0;
    }
    if (d->n != out_features || d->k != in_features) {
        fprintf(stderr, "[s2pro] qcache: cached %s is [%d, %d], the model wants [%d, %d]; "
                        "quantising it live\n", name, d->n, d->k, out_features, in_features);
        return 0;
    }
    uint64_t want_codes, want_scales;
    if (!expected_lengths(d->kind, d->n, d->k, d->group, &want_codes, &want_scales) ||
        want_codes != d->codes_len || want_scales != d->scales_len) {
        fprintf(stderr, "[s2pro] qcache: %s has a malformed descriptor; quantising it live\n", name);
        return 0;
    }
    /* build the linear aside: *lin changes only on a hit */
    s2p_linear got;
    memset(&got, 0, sizeof(got));
    got.in_features = in_features;
    got.out_features = out_features;
    s2p_tensor* codes = d->kind == 2 ? &got.w_pack : &got.w_int8;
    const int64_t cshape[2] = {d->n, (int64_t)(d->codes_len / (uint64_t)d->n)};
    const int64_t sshape[1] = {(int64_t)(d->kind == 1 ? d->scales_len / 4 : d->scales_len / 2)};
    int ok = s2p_tensor_device_alloc(codes, S2P_DT_I8, 2, cshape) == S2P_OK &&
             s2p_tensor_device_alloc(&got.w_iscale, d->kind == 1 ? S2P_DT_F32 : S2P_DT_F16, 1,
                                     sshape) == S2P_OK &&
             codes->bytes == d->codes_len && got.w_iscale.bytes == d->scales_len;
    ok = ok && stream_payload(qc, d->codes_at, d->codes_len, codes->data, stream) &&
         stream_payload(qc, d->scales_at, d->scales_len, got.w_iscale.data, stream);
    if (!ok) {
        fprintf(stderr, "[s2pro] qcache: reading %s failed; quantising it live\n", name);
        (void)drain_staging(qc);
        s2p_tensor_free(codes);
        s2p_tensor_free(&got.w_iscale);
        return 0;
    }
    got.int8_ready = 1;
    got.q_group = d->kind == 1 ? 0 : d->group;
    got.q_packed = d->kind == 2;
    *lin = got;
    return 1;
}

/* --------------------------------------------------------------- write */

static int spool_bytes(s2p_qcache* qc, const void* p, size_t n) {
    if (n && fwrite(p, 1, n, qc->spool) != n) return 0;
    qc->spool_len += n;
    return 1;
}

/* zero-pad the spool to the payload alignment, then device bytes src */
static int spool_device(s2p_qcache* qc, const void* src, uint64_t len, unsigned char* bounce,
                        uint64_t* at) {
    static const unsigned char zeros[PAYLOAD_ALIGN];
    const uint64_t pad = round_up(qc->spool_len) - qc->spool_len;
    if (!spool_bytes(qc, zeros, (size_t)pad)) return 0;
    *at = qc->spool_len;
    for (uint64_t done = 0; done < len;) {
        const size_t n = (size_t)(len - done < CHUNK_BYTES ? len - done : CHUNK_BYTES);
        if (hipMemcpy(bounce, (const unsigned char*)src + done, n, hipMemcpyDeviceToHost) !=
            hipSuccess)
            return -1;
        if (!spool_bytes(qc, bounce, n)) return 0;
        done += n;
    }
    return 1;
}

s2p_status s2p_qcache_put_linear(s2p_qcache* qc, const char* name, const s2p_linear* lin,
                                 hipStream_t stream) {
    if (!qc || qc->reading || qc->spool_failed || !name || !lin || !lin->int8_ready)
        return S2P_OK;
    const size_t name_len = strlen(name);
    const uint32_t kind = lin->q_packed ? 2u : lin->q_group > 0 ? 3u : 1u;
    const s2p_tensor* codes = kind == 2 ? &lin->w_pack : &lin->w_int8;
    if (name_len == 0 || name_len > MAX_NAME || !codes->data || !lin->w_iscale.data)
        return S2P_OK;
    if (qc->count == MAX_DESCS) {
        fprintf(stderr, "[s2pro] qcache: more than %d tensors; %s stays uncached\n", MAX_DESCS,
                name);
        return S2P_OK;
    }
    if (!qc->spool) {
        snprintf(qc->spool_path, sizeof(qc->spool_path), "%s.spool", qc->file);
        qc->spool = fopen(qc->spool_path, "w+b");
        if (!qc->spool) {
            fprintf(stderr, "[s2pro] qcache: cannot create %s; no cache this run\n",
                    qc->spool_path);
            qc->spool_failed = 1;
            return S2P_OK;
        }
    }
    qc_desc d = {0};
    d.kind = kind;
    d.n = lin->out_features;
    d.k = lin->in_features;
    d.group = lin->q_group;
    d.codes_len = codes->bytes;
    d.scales_len = lin->w_iscale.bytes;
    d.name = strdup(name);
    unsigned char* bounce = (unsigned char*)malloc(CHUNK_BYTES);
    if (!d.name || !bounce) {
        free(d.name);
        free(bounce);
        return S2P_OK; /* only the cache degrades */
    }
    /* the tensors were produced on `stream` */
    int r = hipStreamSynchronize(stream) == hipSuccess ? 1 : -1;
    if (r == 1) r = spool_device(qc, codes->data, d.codes_len, bounce, &d.codes_at);
    if (r == 1) r = spool_device(qc, lin->w_iscale.data, d.scales_len, bounce, &d.scales_at);
    free(bounce);
    if (r != 1) {
        free(d.name);
        qc->spool_failed = 1; /* the spool is now inconsistent: drop the cache */
        fprintf(stderr, "[s2pro] qcache: could not spool %s; no cache this run\n", name);
        return r < 0 ? S2P_ERR_CUDA : S2P_OK;
    }
    qc->desc[qc->count++] = d;
    return S2P_OK;
}

static void drop_spool(s2p_qcache* qc) {
    if (qc->spool) {
        fclose(qc->spool);
        qc->spool = NULL;
        remove(qc->spool_path);
    }
}

/* header + table (offsets made absolute) + the spooled payloads -> a
 * temporary file, renamed over the cache */
static int publish(s2p_qcache* qc) {
    uint64_t table_end = HEAD_BYTES;
    for (int i = 0; i < qc->count; i++) table_end += DESC_BYTES + strlen(qc->desc[i].name);
    const uint64_t base = round_up(table_end);
    unsigned char* head = (unsigned char*)calloc(1, (size_t)base);
    unsigned char* buf = (unsigned char*)malloc(CHUNK_BYTES);
    int ok = head && buf && fflush(qc->spool) == 0;
    if (ok) {
        memcpy(head, k_magic, sizeof(k_magic));
        put_u64(head + 8, qc->stamp);
        put_u32(head + 16, (uint32_t)qc->count);
        unsigned char* w = head + HEAD_BYTES;
        for (int i = 0; i < qc->count; i++) {
            const qc_desc* d = &qc->desc[i];
            const uint32_t nl = (uint32_t)strlen(d->name);
            put_u32(w, nl);
            put_u32(w + 4, d->kind);
            put_u32(w + 8, (uint32_t)d->n);
            put_u32(w + 12, (uint32_t)d->k);
            put_u32(w + 16, (uint32_t)d->group);
            put_u64(w + 24, base + d->codes_at);
            put_u64(w + 32, d->codes_len);
            put_u64(w + 40, base + d->scales_at);
            put_u64(w + 48, d->scales_len);
            memcpy(w + DESC_BYTES, d->name, nl);
            w += DESC_BYTES + nl;
        }
    }
    char part[1100];
    snprintf(part, sizeof(part), "%s.part", qc->file);
    FILE* out = ok ? fopen(part, "wb") : NULL;
    ok = out && fwrite(head, 1, (size_t)base, out) == (size_t)base;
    const int sfd = fileno(qc->spool);
    for (uint64_t at = 0; ok && at < qc->spool_len;) {
        const size_t n = (size_t)(qc->spool_len - at < CHUNK_BYTES ? qc->spool_len - at : CHUNK_BYTES);
        ok = pread_all(sfd, buf, n, at) && fwrite(buf, 1, n, out) == n;
        at += n;
    }
    if (out) ok = fclose(out) == 0 && ok;
    ok = ok && rename(part, qc->file) == 0;
    if (!ok) remove(part);
    free(head);
    free(buf);
    return ok;
}

/* ------------------------------------------------------------ lifecycle */

s2p_status s2p_qcache_open(const char* model_dir, s2p_gemm_mode mode, s2p_qcache** out) {
    if (!model_dir || !out) return S2P_ERR_INVALID;
    *out = NULL;
    /* only the INT8 / INT4 modes carry quantised tensors */
    if (mode != S2P_GEMM_INT8 || !switch_on("S2P_QCACHE", 1)) return S2P_OK;
    uint64_t stamp;
    if (weights_stamp(model_dir, mode, &stamp) != 0) return S2P_OK; /* no weights: no cache */
    s2p_qcache* qc = (s2p_qcache*)calloc(1, sizeof(*qc));
    if (!qc) return S2P_ERR_OOM;
    qc->stamp = stamp;
    qc->fd = -1;
    const char* dir = getenv("S2P_QCACHE_DIR");
    snprintf(qc->file, sizeof(qc->file), "%s/s2p_qcache.bin", dir && *dir ? dir : model_dir);
    qc->fd = open(qc->file, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (qc->fd >= 0 && fstat(qc->fd, &st) == 0) {
        qc->file_len = (uint64_t)st.st_size;
        qc->reading = load_table(qc);
    }
    if (qc->reading) {
        fprintf(stderr, "[s2pro] qcache: loading %d quantised tensors from %s\n", qc->count,
                qc->file);
    } else {
        if (qc->fd >= 0) close(qc->fd);
        qc->fd = -1;
        fprintf(stderr, "[s2pro] qcache: no usable cache; %s will be written after loading\n",
                qc->file);
    }
    *out = qc;
    return S2P_OK;
}

int s2p_qcache_reading(const s2p_qcache* qc) { return qc && qc->reading; }

s2p_status s2p_qcache_finish(s2p_qcache* qc, hipStream_t stream) {
    (void)stream; /* the uploads are tracked by their own events */
    if (!qc) return S2P_OK;
    if (qc->reading) {
        const int ok = drain_staging(qc);
        release_reader(qc);
        return ok ? S2P_OK : S2P_ERR_CUDA;
    }
    if (qc->spool && !qc->spool_failed && qc->count > 0) {
        if (publish(qc))
            fprintf(stderr, "[s2pro] qcache: stored %d quantised tensors in %s\n", qc->count,
                    qc->file);
        else
            fprintf(stderr, "[s2pro] qcache: writing %s failed; no cache this run\n", qc->file);
    }
    drop_spool(qc);
    return S2P_OK;
}

void s2p_qcache_free(s2p_qcache* qc) {
    if (!qc) return;
    release_reader(qc);
    drop_spool(qc);
    forget_descs(qc);
    free(qc);
}
