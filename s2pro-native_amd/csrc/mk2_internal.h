/* s2pro MI355X — descriptor of the persistent verify kernel (mk2.hip),
 * shared with the C host code (verify.c).  Not public ABI. */
#ifndef S2P_MK2_INTERNAL_H
#define S2P_MK2_INTERNAL_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#include "prims_internal.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Tile-packed INT4-g32 weights: a 16-row tile's 4-group block is 1152 B:
 * 1024 B of codes (lane l = quarter q = l / 16, row r = l % 16: 16 B = one
 * dword per group, the row's k = 8q..8q+7 of that group, nibbles biased by
 * +8 and placed so that dword >> 4j & 0x000F000F holds k = 8q+2j, 8q+2j+1)
 * then 128 B of f16 scales [16 rows][4 groups].  A linear is [tile][block];
 * gate_up's tile t holds gate rows 8t..8t+7 (tile rows 0..7) and the
 * matching up rows (tile rows 8..15): 1216 tiles, 8 h columns each. */
#define MK2_BLK 1152
#define MK2_MAX_ROWS 6    /* rows the kernel serves (the w2 activations fill LDS) */
#define MK2_NWG 256       /* one workgroup per CU of an MI355X */

/* per-layer packed block counts and offsets (blocks) */
#define MK2_BLK_Q (384 * 20)
#define MK2_BLK_O (160 * 32)
#define MK2_BLK_G (1216 * 20)
#define MK2_BLK_D (160 * 76)
#define MK2_LAYER_BLKS (MK2_BLK_Q + MK2_BLK_O + MK2_BLK_G + MK2_BLK_D)

/* per-layer norm weights, packed: attn 2560 | ffn 2560 | q 128 | k 128 */
#define MK2_NORM_ATTN 0
#define MK2_NORM_FFN 2560
#define MK2_NORM_Q 5120
#define MK2_NORM_K 5248
#define MK2_NORM_STRIDE 5376

/* flags: one 32-bit word per producing workgroup (GEMV phases, the init) or
 * attention unit, each in its own 64-byte line (MK2_FSTR words apart: flags
 * sharing a line made every hop ~1.4 us slower, the writers and the pollers
 * of all workgroups contending for the same lines); offsets in words */
#define MK2_FSTR 16
#define MK2_F_INIT 0                          /* 256 workgroups */
#define MK2_F_Q (256 * MK2_FSTR)              /* 256 workgroups */
#define MK2_F_ATT (512 * MK2_FSTR)            /* n_seg x 8 x nsplit units (<= 3072) */
#define MK2_F_O ((512 + 3072) * MK2_FSTR)     /* 256 workgroups */
#define MK2_F_G ((768 + 3072) * MK2_FSTR)     /* 256 workgroups */
#define MK2_F_D ((1024 + 3072) * MK2_FSTR)    /* 256 workgroups */
#define MK2_F_PART ((1280 + 3072) * MK2_FSTR) /* attention units: their split partials written */
#define MK2_F_WORDS ((1280 + 2 * 3072) * MK2_FSTR)
#define MK2_ATT_MAX 3072
#define MK2_MAX_LAYERS 40
#define MK2_MAX_SPLIT 64
/* default polls of one flag wait before it gives up (seconds, not a schedule) */
#define MK2_SPIN_LIMIT (1u << 22)
/* the backbone's mk2 state block (uint32 words): flags, then the launch
 * epoch and done count, the error flag.  Zeroed at every plan; within a
 * plan every word only grows. */
#define MK2_STATE_WORD MK2_F_WORDS
#define MK2_ERR_WORD (MK2_STATE_WORD + 2)
#define MK2_STATE_WORDS (MK2_STATE_WORD + 4)
/* after the state block (256-aligned): the norm-weighted residual rows
 * [MK2_MAX_ROWS][2560] bf16 and the code-bias terms of the GEMV inputs,
 * -136 x (sum of a row's values), f32, [column block][8 rows] (rows >= the
 * plan's rows stay 0): weighted residual [160][8] per 16 columns, h [304][2][8] per 32
 * columns, attention output [128][8] per 32 columns.  Zeroed at every plan. */
#define MK2_AUX_OFF (((MK2_STATE_WORDS * 4 + 255) / 256) * 256)
#define MK2_AUX_XW 0
#define MK2_AUX_GSX (MK2_AUX_XW + MK2_MAX_ROWS * 2560 * 2)
#define MK2_AUX_GSH (MK2_AUX_GSX + 160 * 8 * 4)
#define MK2_AUX_GSA (MK2_AUX_GSH + 608 * 8 * 4)
#define MK2_AUX_BYTES (MK2_AUX_GSA + 128 * 8 * 4)

typedef struct {
    const uint8_t* wpack;          /* [n_layers][MK2_LAYER_BLKS] packed blocks */
    const uint8_t* hpack;          /* head [head_tiles][20] */
    int head_tiles, head_n;        /* tiles (rows padded to 16) and real rows */
    const uint16_t* norms;         /* [n_layers][MK2_NORM_STRIDE]: attn, ffn, q, k norm weights */
    const uint16_t* final_norm;
    int n_layers, rows;
    const uint16_t* x_in;
    uint16_t* x;                   /* [rows][2560] residual stream */
    uint16_t* qkv;                 /* [rows][6144] */
    uint16_t* q;                   /* [rows][4096] (inspection copy of the roped q rows) */
    uint16_t* attn;                /* [rows][4096] */
    uint16_t* h;                   /* [rows][9728] */
    uint16_t* logits;              /* [rows][head_n] */
    float* ssq;                    /* [MK2_MAX_ROWS][160] per-16-column sums of squares of x */
    uint16_t* xw;                  /* [rows][2560] bf16(x * the next RMSNorm's weight) */
    float* gsx;                    /* [160][8] code-bias terms of xw per 16 columns */
    float* gsh;                    /* [304][2][8] of h per 32 columns, in two parts: part 1
                                      from a workgroup the group did not begin in (else 0) */
    float* gsa;                    /* [128][8] of attn per 32 columns */
    uint32_t* flags;               /* [MK2_F_KINDS][MK2_F_STRIDE] */
    uint32_t* state;               /* [0] launch epoch, [1] workgroups done (monotonic) */
    int* err;                      /* sticky: a wait timed out */
    unsigned spin_limit;           /* polls per flag wait before it gives up */
    int kvb;                       /* session caches: 16 = bf16; 8 / 4 = INT8 / INT4 codes
                                    * [layers][16][ctx][128 / 64] with f16 group scales
                                    * [layers][16][ctx][4] behind plan.kvs
                                    * (slowar_internal.h:177-179) */
    /* attention */
    S2pRowPlan plan;
    const S2pAttnSeg* segs;
    int n_seg, nsplit, split_pos;
    float* attn_part;
    const float* rope_tab;
    float eps;
} Mk2Args;

/* 0 when the device can run the kernel (MK2_NWG co-resident workgroups) */
int s2p_mk2_supported(void);
/* pack one INT4-g32 linear (codes [N][K/2], f16 scales [N][K/32]) into the
 * tile layout at dst; pairs = 1: rows [0, N/2) gate, [N/2, N) up */
hipError_t s2p_mk2_pack(const void* w_pack, const void* scales, int N, int K, int pairs,
                        void* dst, hipStream_t st);
/* args: host copy, passed by value (kernel arguments) */
hipError_t s2p_mk2_launch(const Mk2Args* args, hipStream_t st);

#ifdef __cplusplus
}
#endif
#endif
