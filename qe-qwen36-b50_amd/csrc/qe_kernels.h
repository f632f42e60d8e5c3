// Kernel argument blocks and host launchers of the MoE block (internal).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qe_device.h"

#define QE_SMALL_T 8   /* calls of up to this many tokens take the persistent decode kernel */
#define RT_SPLIT 8     /* router K split: subtrees of 64 / RT_SPLIT chunks, merged by k_topk */
#define QE_MFMA_MC 64 /* pairs per work item of the prefill MFMA grouped GEMMs (up to four 16-row tiles) */


// One layer's weights inside the context.
struct QeLayerPtrs {
    const uint8_t *arena;     // 256 expert blobs
    const float *router;      // [257][2048]
    const float *bias;        // [256] or nullptr
    const uint8_t *sh_gu;     // Q8 [1024][2048]
    const uint8_t *sh_dn;     // Q8 [2048][512]
    const float *post_norm;   // [2048]
};

// Optional per-kernel event timing (host side): when `on`, every launch of
// qe_launch_layer is bracketed by two events on its stream.
enum { QP_DECODE, QP_NORMQ, QP_ROUTER, QP_SHGU, QP_TOPK, QP_DISPATCH, QP_GU, QP_HQUANT, QP_DOWN_LARGE, QP_SHDN,
       QP_COMBINE, QP_N };
struct QeProf {
    bool on = false;
    int used = 0, cap = 0, dropped = 0;
    hipEvent_t *ev = nullptr; // 2*cap events
    int *kid = nullptr;       // kernel id per pair
};

// Event bracket of one launch when per-kernel timing is on.
struct ProfScope {
    QeProf *p;
    hipStream_t st;
    int slot = -1;
    ProfScope(QeProf *p_, int kid, hipStream_t s) : p(p_), st(s) {
        if (!p || !p->on) return;
        if (p->used >= p->cap) { p->dropped++; return; }
        slot = p->used++;
        p->kid[slot] = kid;
        (void)hipEventRecord(p->ev[2 * slot], st);
    }
    ~ProfScope() {
        if (slot >= 0) (void)hipEventRecord(p->ev[2 * slot + 1], st);
    }
};

// Scratch of a context, sized for t_max tokens.
struct QeScratch {
    float *xn; int8_t *xqp; float *xs;      // [T][2048] normed x, its int8 quantisation (operand layout), [T][64] scales
    _Float16 *xhl;                          // [T][2048] normed x as fp16 hi|lo halves (store_hilo16 layout)
    float *logits;                          // [T][257]
    float *shgu;                            // prefill: shared silu(g)*u as [T][512] fp16 hi|lo halves
    float *rpart;                           // [8][T][256] router subtree partials
    int32_t *ids; float *wts; float *shg;   // [T][8], [T][8], [T]
    int32_t *off; int32_t *pairs;           // [257], [T*8]
    int4 *items; int32_t *n_items;          // work items (expert, first pair, count); n_items[0] items, the first n_items[1] big
    int8_t *hqp; float *hs;                 // [T*8][512] quantised h (operand layout), [T*8][16] scales
    float *sd;                              // [T][2048] shared-expert output
    float *yp;                              // [T*8][2048] weighted expert outputs
    int32_t *chunk_hist;                    // [T*8/1024][256]
    int32_t *item_done;                     // [max items] finished gate/up workgroups per item (fused launch)
    unsigned *err; unsigned err_val;        // a fused launch's wait that gave up stores err_val to *err
    int spin_cap;                           // reads such a wait may take
    int wait_extra;                         // test hook: gate/up workgroups a fused down wait expects beyond its item's
    int t_max;
    QeProf *prof;                           // host-side timing, may be nullptr
};

struct QeCombineArgs {
    int T;
    const float *yp; const float *sd; const float *shg; const float *x2;
    float *out;
    const float *nw; float *xn; // optional exit norm: xn = RMSNorm(out) * nw (nw == nullptr: none)
};

// Persistent decode kernel (qe_decode.hip): T <= QE_SMALL_T tokens through
// layers first_layer .. first_layer + n_layers - 1 in one cooperative launch.
struct QeDecodeArgs {
    const uint8_t *arena; const float *router; const float *bias; const uint8_t *bias_on;
    const uint8_t *sh_gu; const uint8_t *sh_dn; const float *post_norm;
    int first_layer, n_layers, T, norm, residual;
    const float *x_in; float *x_out;
    uint64_t *ex;        // exchange words {value, tag}, QE_DECODE_EX_WORDS of them (qe_decode.hip)
    // routing sink of the last layer (plain stores by workgroup 0)
    float *logits; int32_t *ids; float *wts; float *shg; int32_t *off; int32_t *pairs; float *sd_out; float *xn_out;
    unsigned *sync;      // QE_DECODE_SYNC_WORDS: [0] launch epoch, [32] exit counter
    unsigned *err;       // host-mapped: set to 1 + epoch when a poll of the launch timed out
    int spin_cap;        // reads an exchange poll makes before it gives up (QE_DECODE_SPIN_CAP)
    const float *exit_norm; float *exit_xn; // optional: exit_xn = RMSNorm(x_out) * exit_norm
};
hipError_t qe_launch_decode(const QeDecodeArgs &a, hipStream_t st);
#ifndef QE_DEC_REP
#define QE_DEC_REP 4 /* copies of every decode exchange buffer */
#endif
#define QE_DECODE_EX_WORDS \
    (QE_DEC_REP * (2 * QE_SMALL_T * QE_D + QE_SMALL_T * QE_ROUTER_ROWS + QE_SMALL_T * QE_FF_SH + QE_SMALL_T * 8 * 16 * 9 + \
                   8 * QE_FF_EXP + 2 * QE_SMALL_T * 256))
#define QE_DECODE_SYNC_WORDS 64 /* launch epoch, exit counter */
#define QE_DECODE_SPIN_CAP (1 << 22) /* poll reads (s_sleep 1 between) before an exchange wait gives up */
#define QE_DECODE_SPIN_CAP_LATE 16  /* the cap of a wave's polls after one of them gave up */

// Launchers (qe_kernels.hip).  xin: layer input; post_norm: nullptr = input is
// already normalised; x2: residual added to the output or nullptr.
// tokens of the largest call (the API's limit): the down epilogue's 32-bit store
// offsets rely on its pair count staying below 2^19
#define QE_LAYER_T_MAX 65536
hipError_t qe_launch_layer(const QeLayerPtrs &L, const QeScratch &S, const float *xin, bool norm, const float *x2,
                           float *out, int T, hipStream_t st, const float *exit_norm = nullptr,
                           float *exit_xn = nullptr);
hipError_t qe_launch_dispatch(const QeScratch &S, int T, hipStream_t st);
// The same dispatch with its scratch in a static device array (no allocation);
// off and pairs are the caller's device buffers.
#define QE_DISPATCH_NOALLOC_T_MAX 16384
hipError_t qe_launch_dispatch_noalloc(const int32_t *ids, int T, int32_t *off, int32_t *pairs, hipStream_t st);
// the current device's address of that array, looked up once per device
hipError_t qe_noalloc_prepare(uint8_t **base);
hipError_t qe_launch_expert_mfma(const QeLayerPtrs &L, const QeScratch &S, int T, hipStream_t st);
hipError_t qe_launch_router_shgu(const QeLayerPtrs &L, const QeScratch &S, int T, hipStream_t st);

// IQ4_NL conversion (qe_convert.hip): block g (of nblk, nb per row) of the
// source goes to row g / nb of the destination, rows grouped rows_per_group
// at a time (one expert's matrix) at group_stride, row_stride within a group.
struct QeNl4Args {
    const uint8_t *src; uint8_t *dst;
    uint32_t nblk, nb, rows_per_group;
    size_t group_stride, row_stride;
};
hipError_t qe_launch_nl4_quant(const QeNl4Args &a, int src_type, hipStream_t st);

hipError_t qe_launch_synth_layer(uint8_t *arena_l, float *router_l, uint8_t *sh_gu_l, uint8_t *sh_dn_l,
                                 float *post_norm_l, uint64_t seed, int layer, hipStream_t st);
hipError_t qe_launch_synth_x(float *out, uint64_t seed, int inst, int64_t n, hipStream_t st);
