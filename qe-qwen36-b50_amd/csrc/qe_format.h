// Weight-row formats and model constants of the Qwen3.6-35B-A3B MoE block.
//
// Byte layouts are fixed by the reference pack format so that a real pack's
// `blk.N.experts` blob copies into the expert arena unchanged
// (reference engine/pack.h:10-42):
//   * NL4 (IQ4_NL) row of c columns: c/2 bytes of 4-bit codebook indices, then
//     c/32 fp16 scales.  Per 32-weight block, 16 bytes: byte j holds element j
//     in its low nibble and element j+16 in its high nibble (pack.h:27).
//   * Q8 row of c columns: c int8 values, then c/32 fp16 scales (pack.h:24).
//   * Expert blob: gate rows 0..511 (NL4, 2048 cols), up rows 0..511, then down
//     rows 0..2047 (NL4, 512 cols) (pack.h:39-42).
// This header is plain C so it compiles in the HIP library, the C++ host code
// and the CPU oracle alike.
#pragma once
#include <stddef.h>
#include <stdint.h>

#define QE_D 2048         /* hidden size (pack.h:11) */
#define QE_N_EXPERT 256   /* routed experts per layer (pack.h:12) */
#define QE_K_USED 8       /* experts per token (pack.h:12) */
#define QE_FF_EXP 512     /* routed expert intermediate size (pack.h:12) */
#define QE_FF_SH 512      /* shared expert intermediate size (pack.h:12) */
#define QE_N_LAYER 40     /* layers of the model (pack.h:11) */
#define QE_BLK 32         /* weights per quantization block */
#define QE_RMS_EPS 1e-6f  /* pack.h:19 */

/* NL4 row bytes: D=2048 cols -> 1024 code bytes + 64 scales = 1152 B. */
#define QE_NL4_ROW_BYTES(cols) ((size_t)(cols) / 2 + (size_t)(cols) / QE_BLK * 2)
/* Q8 row bytes: 2048 cols -> 2048 + 128 = 2176 B. */
#define QE_Q8_ROW_BYTES(cols) ((size_t)(cols) + (size_t)(cols) / QE_BLK * 2)

#define QE_GU_ROW_BYTES QE_NL4_ROW_BYTES(QE_D)      /* 1152 */
#define QE_DN_ROW_BYTES QE_NL4_ROW_BYTES(QE_FF_EXP) /* 288 */
#define QE_EXPERT_BYTES \
    (2 * (size_t)QE_FF_EXP * QE_GU_ROW_BYTES + (size_t)QE_D * QE_DN_ROW_BYTES) /* 1,769,472 */
#define QE_EXPERT_DOWN_OFF (2 * (size_t)QE_FF_EXP * QE_GU_ROW_BYTES)          /* 1,179,648 */
#define QE_LAYER_EXPERT_BYTES ((size_t)QE_N_EXPERT * QE_EXPERT_BYTES)         /* 452,984,832 */

#define QE_SH_GU_ROWS (2 * QE_FF_SH)                      /* gate rows 0..511, up rows 512..1023 */
#define QE_SH_GU_ROW_BYTES QE_Q8_ROW_BYTES(QE_D)          /* 2176 */
#define QE_SH_DN_ROW_BYTES QE_Q8_ROW_BYTES(QE_FF_SH)      /* 544 */
#define QE_SH_GU_BYTES ((size_t)QE_SH_GU_ROWS * QE_SH_GU_ROW_BYTES) /* 2,228,224 */
#define QE_SH_DN_BYTES ((size_t)QE_D * QE_SH_DN_ROW_BYTES)          /* 1,114,112 */
#define QE_ROUTER_ROWS (QE_N_EXPERT + 1)                  /* row 256 = shared-expert gate */
#define QE_ROUTER_BYTES ((size_t)QE_ROUTER_ROWS * QE_D * 4)         /* 2,105,344 */

/* IQ4_NL codebook (pack.h:37). */
static const int8_t QE_KVALUES_NL4[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                          1,    13,   25,  38,  53,  69,  89,  113};
/* The same codebook packed four entries per dword (entry i in byte i%4 of
 * word i/4), the operand form a byte-permute lookup wants. */
#define QE_NL4_W0 0xBFAD9881u /* -127 -104  -83  -65 */
#define QE_NL4_W1 0xF6EADDCFu /*  -49  -35  -22  -10 */
#define QE_NL4_W2 0x26190D01u /*    1   13   25   38 */
#define QE_NL4_W3 0x71594535u /*   53   69   89  113 */
