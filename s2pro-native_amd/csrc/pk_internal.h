/* s2pro MI355X — descriptors of the persistent verify kernel (verify_pk.hip),
 * shared with the C host code (verify.c).  Not public ABI.
 *
 * One launch runs the whole K-token verify forward (36 layers + lm head) for
 * one session of M <= PK_MAXM rows over a bf16 cache with INT4-g32 weights.
 * Every CU runs one workgroup: PK_CW compute waves and one loader wave.  The
 * loader streams the CU's share of every weight matrix of the step, in the
 * order the compute waves consume it, into a ring of LDS slots (direct-to-LDS
 * loads); the weights were repacked once into one contiguous stream per CU
 * (s2p_pk_repack), so the loader's reads are sequential and independent of
 * the activations, and it runs ahead of the phase barriers. */
#ifndef S2P_PK_INTERNAL_H
#define S2P_PK_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_CW 8                       /* compute waves per workgroup */
#define PK_THREADS (64 * (PK_CW + 1)) /* + the loader wave */
#define PK_CHUNK 1152                 /* one stream chunk: 16 rows x 4 groups of INT4 (1 KiB) + their f16 scales */
#define PK_SLOTS 40                   /* ring slots (a multiple of PK_CW) */
#define PK_MAXM 7                     /* rows per launch (activation blocks hold 8 rows; row 7 carries sums of squares) */
#define PK_MAX_SPLITS 32              /* attention position splits per kv head */
#define PK_PART_STRIDE 132            /* floats per partial: max, sum, 128 dims (+2 pad) */
#define PK_HEAD_MAX_TILES 64          /* head tiles per CU (wave-tile mode) */

/* a GEMV of the stream: N output rows (SwiGLU: 2F, gate rows then up rows),
 * K inputs; tiles (SwiGLU: gate/up tile pairs) are dealt to the CUs in
 * contiguous ranges [c*T/ncu, (c+1)*T/ncu) */
enum { PK_G_WQKV = 0, PK_G_WO = 1, PK_G_GU = 2, PK_G_W2 = 3 };

/* an activation block: 16 columns x 8 rows bf16 (256 B, one writer); rows
 * 0..M-1 hold values, row 7 of a residual block holds the rows' sums of
 * squares over the block's 16 columns as f32 */
#define PK_BLK 256

typedef struct {
    /* weights */
    const uint8_t* stream;    /* repacked chunks, CU after CU */
    const int64_t* cu_chunk0; /* [ncu] first chunk of each CU's stream */
    int n_layers;
    int head_rows;            /* rows of the lm head (16-row tiles) */
    const uint16_t* const* attn_norm; /* [n_layers] bf16 [2560] */
    const uint16_t* const* ffn_norm;
    const uint16_t* const* q_norm;    /* [n_layers] bf16 [128] */
    const uint16_t* const* k_norm;
    const uint16_t* final_norm;
    float eps;
    /* activations, one buffer per (layer, producer): written once per launch */
    uint16_t* xb;   /* [2 n_layers + 1][160 blocks]: x before layer l (2l), after its wo (2l+1) */
    uint16_t* qkvb; /* [n_layers][384 blocks] */
    uint16_t* ob;   /* [n_layers][256 blocks] attention outputs */
    uint16_t* hb;   /* [n_layers][608 blocks] SwiGLU outputs */
    float* part;    /* [n_layers][8 kv heads][PK_MAX_SPLITS][PK_MAXM * 4][PK_PART_STRIDE] */
    /* plan (one session) */
    int M, L;                 /* rows; cached prefix length (row i writes slot L + i) */
    int pos[PK_MAXM];         /* RoPE positions */
    uint64_t vis[PK_MAXM];    /* visible node slots relative to L (bit i: slot L + i) */
    uint16_t* kv;             /* session KV base [layers][16][max_seq][128] bf16 */
    int64_t layer_stride;     /* elements per layer */
    int max_seq;
    const float* rope_tab;    /* [M][64][cos, sin] */
    int nsplit, split_pos;    /* attention position splits per kv head */
    /* synchronisation */
    uint32_t* flags;          /* [ncu] barrier arrival epochs (monotonic across launches) */
    int* err;                 /* sticky: a bounded wait ran out */
} PkArgs;

/* grid of the kernel: workgroups (= CUs) and dynamic LDS bytes; 0 on success */
int s2p_pk_grid(int* nwg, size_t* lds);
/* chunks of the stream of CU c of ncu for a backbone of n_layers and head rows */
int64_t s2p_pk_cu_chunks(int c, int ncu, int n_layers, int head_rows);
/* repack one GEMV (kind PK_G_*, or 4 = the head) of layer l into the streams:
 * w packed INT4 [N][K/2] (two's complement nibbles, low nibble = even k), s f16
 * [N][K/32]; stream / cu_chunk0 as in PkArgs (device) */
hipError_t s2p_pk_repack(uint8_t* stream, const int64_t* cu_chunk0_dev, int ncu, int n_layers,
                         int head_rows, int layer, int kind, const uint8_t* w, const uint16_t* s,
                         int N, int K, hipStream_t st);
hipError_t s2p_pk_launch(const PkArgs* args_dev, const void* x_in, void* logits, int nwg,
                         size_t lds, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
