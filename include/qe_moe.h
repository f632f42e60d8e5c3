/* qe_moe.h -- C ABI of the MI355X (gfx950) Qwen3.6-35B-A3B MoE block.
 *
 * One context owns, on one GPU, a flat expert arena holding every routed
 * expert of every layer (n_layers x 256 blobs in the reference pack layout),
 * the per-layer dense weights (post-norm, router + shared-gate rows, Q8 shared
 * expert) and all scratch for up to t_max tokens per call.  It replaces the
 * MoE sections of the reference engine:
 *   Engine::moe_batched ........... engine/qe.cpp:1957-2047 (prefill / chunks)
 *   MoE block of Engine::decode ... engine/qe.cpp:2466-2572 (B = 1)
 *   MoE block of decode_multi<NT> . engine/qe.cpp:1653-1737 (NT <= 8)
 * and the VRAM/RAM expert residency tables (engine/qe.cpp:927-931,
 * 1131-1198), which become the flat arena: expert e of layer l lives at
 * arena + (l*256 + e) * qe_moe_expert_bytes().
 *
 * Conventions: plain pointers and sizes; activations are device pointers to
 * fp32 [T][2048] row-major; `stream` is a hipStream_t (NULL = default
 * stream).  Calls enqueue work on `stream` and return without a host sync,
 * except qe_moe_get_routing, which copies to the host.  A context is used by
 * one host thread at a time, and calls on one context must not overlap on
 * different streams (the reference's single-engine-thread rule,
 * engine/qe.cpp:877, 3162).  Every entry point returns 0 or a negative
 * QE_ERR_* code; qe_moe_last_error() describes the last failure of the
 * calling thread.  The reference has no error returns (it exits,
 * engine/qe.cpp:1022); these codes replace that.
 */
#ifndef QE_MOE_H
#define QE_MOE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QE_OK 0
#define QE_ERR_ARG (-1)   /* bad argument (null pointer, layer or T out of range) */
#define QE_ERR_HIP (-2)   /* a HIP runtime call failed */
#define QE_ERR_OOM (-3)   /* device allocation failed */
#define QE_ERR_STATE (-4) /* layer not ready (a weight tensor or expert never set), or an earlier launch
                              timed out in a bounded wait (see qe_moe_check) */

typedef struct qe_moe_ctx qe_moe_ctx;

/* Largest t_max a context accepts (prefill scratch offsets stay 32-bit). */
#define QE_MOE_T_MAX 65536

/* Create a context on `device` for n_layers layers and calls of up to t_max
 * tokens (1..QE_MOE_T_MAX).  Allocates the arena (n_layers * 452,984,832 B)
 * and scratch.
 * Replaces Engine::Engine's upload/arena/scratch set-up (engine/qe.cpp:1038-1244). */
int qe_moe_create(int device, int n_layers, int t_max, qe_moe_ctx **out);
int qe_moe_destroy(qe_moe_ctx *ctx);

/* Bytes of one routed expert blob: gate[512] | up[512] | down[2048] NL4 rows
 * (engine/pack.h:40-42, exp_bytes()). */
size_t qe_moe_expert_bytes(void);

/* Copy n_experts blobs (expert ids first..first+n-1 of `layer`) into the arena,
 * from host (src_on_device = 0) or device memory.  A pack's blk.N.experts
 * entry (engine/qconv.cpp:202-228) copies in as is.  A host source is copied
 * before the call returns; a device source is copied in `stream` order.
 * Replaces the arena/host expert copies of engine/qe.cpp:1172-1194. */
int qe_moe_upload_experts(qe_moe_ctx *ctx, int layer, int first, int n_experts, const void *src, int src_on_device,
                          void *stream);

/* Set a layer's dense weights (engine/qe.cpp:855-870 Layer fields, uploaded at
 * :1053-1057): post_norm fp32[2048]; router fp32[257][2048] (rows 0..255 the
 * expert router, row 256 the shared-expert gate, as upload({router, sh_gate})
 * builds it at :1055); bias fp32[256] added to logits 0..255 (NULL = none);
 * sh_gu Q8 [1024 rows x 2048] (gate rows 0..511, up rows 512..1023);
 * sh_down Q8 [2048 rows x 512].  Any pointer may be NULL to keep the current
 * contents.  Sources are host or device memory per src_on_device; host
 * sources are copied before the call returns. */
int qe_moe_set_dense(qe_moe_ctx *ctx, int layer, const float *post_norm, const float *router, const float *bias,
                     const void *sh_gu, const void *sh_down, int src_on_device, void *stream);

/* Full MoE section: x = x2 + MoE(RMSNorm(x2) * post_norm), T tokens.
 * Replaces Engine::moe_batched (engine/qe.cpp:1957) and the MoE blocks of
 * decode (:2466-2572) / decode_multi (:1653-1737).  x may not alias x2. */
int qe_moe_forward(qe_moe_ctx *ctx, int layer, const float *x2, float *x, int T, void *stream);

/* As qe_moe_forward, then the next block's input norm on the result:
 * xn = RMSNorm(x) * next_norm (fp32 [2048], device memory), in the same
 * canonical order as the entry norm.  Replaces Engine::moe_batched
 * (engine/qe.cpp:1957) followed by the next layer's
 * rmsnorm_rows(X, attn_norm, XN) (:1280), or by the final out_norm (:1295);
 * in decode, the MoE block (:2466-2572) followed by rmsnorm(x, attn_norm, xn)
 * (:2243) or out_norm (:2574).  xn may not alias x or x2. */
int qe_moe_forward_norm(qe_moe_ctx *ctx, int layer, const float *x2, float *x, int T, const float *next_norm, float *xn,
                        void *stream);

/* MoE on already-normalised input, no residual: y = MoE(xn).  The "one MoE
 * layer" of the benchmark configurations; the same kernels as qe_moe_forward
 * with the norm and the residual switched off. */
int qe_moe_forward_normed(qe_moe_ctx *ctx, int layer, const float *xn, float *y, int T, void *stream);

/* Layers first..first+n_layers-1 in sequence, each x_{l+1} = x_l +
 * MoE_l(RMSNorm(x_l)): the per-layer MoE steps of the decode loop
 * (engine/qe.cpp:2241-2572) with attention/DeltaNet left out.  x_in is not
 * modified; the result lands in x_out; the context's ping-pong buffer holds
 * intermediate layers. */
int qe_moe_forward_stack(qe_moe_ctx *ctx, int first_layer, int n_layers, const float *x_in, float *x_out, int T,
                         void *stream);

/* Routing of the last forward call (synchronises `stream`, copies to host):
 * ids int32[T][8] (k = 0 largest), weights fp32[T][8], shared gate fp32[T],
 * off int32[257] (exclusive per-expert prefix), pairs int32[T*8] (pair
 * p = t*8+k grouped by expert, ascending p inside an expert), shared-expert
 * output fp32[T][2048] before gating.  Any output may be NULL.  The parity
 * sink of the reference's IDB/WB/SHG/PAIRS/OFF/SD buffers (engine/qe.cpp:1966-1978). */
int qe_moe_get_routing(qe_moe_ctx *ctx, int T, int32_t *ids, float *wts, float *shg, int32_t *off, int32_t *pairs,
                       float *shared_out, void *stream);

/* Token-to-expert dispatch alone on caller-supplied ids (device int32[T][8],
 * each in 0..255; the kernels reduce other values modulo 256, so a bad id
 * yields a wrong permutation but no out-of-bounds access): per-expert histogram, exclusive scan and the stable
 * permutation of Engine::moe_batched (engine/qe.cpp:1965-1976), run on the
 * GPU; read the result with qe_moe_get_routing (off, pairs). */
int qe_moe_dispatch(qe_moe_ctx *ctx, const int32_t *ids, int T, void *stream);

/* qe_moe_dispatch without a context and without allocating: the same
 * histogram / scan / stable permutation (results identical to
 * qe_moe_dispatch followed by qe_moe_get_routing's off and pairs), written to
 * the caller's device buffers off int32[257] and pairs int32[T*8], on the
 * calling thread's current device.  No reference counterpart: it is for
 * callers that cannot call hipMalloc (code under HIP graph capture, tight
 * serving loops, harnesses that forbid allocation).  Its scratch (chunk
 * histograms and work items, about 200 KB) is a static device array the
 * library holds on every device it runs on until the process ends, sized for
 * T <= QE_MOE_DISPATCH_NOALLOC_T_MAX; larger T returns QE_ERR_ARG.  Every call
 * on one device shares that array: calls that overlap on one device (other
 * streams, other threads) race.  Under HIP graph capture: the array's address
 * on a device is looked up once, by qe_moe_create for its device or else by
 * the first call on that device, and the lookup must not run while a stream
 * is capturing: create a context on the device, or make one call, before
 * capturing the first one. */
#define QE_MOE_DISPATCH_NOALLOC_T_MAX 16384
int qe_moe_dispatch_noalloc(const int32_t *ids, int T, int32_t *off, int32_t *pairs, void *stream);

/* Router logits fp32[T][257] of the last forward call (synchronises `stream`,
 * copies to host): the parity sink of the reference's RL buffer
 * (engine/qe.cpp:1959). */
int qe_moe_get_logits(qe_moe_ctx *ctx, int T, float *logits, void *stream);

/* Per-kernel timing, the counterpart of the reference's QE_PROF phase timers
 * (engine/qe.cpp:1246-1251; MoE phases at :1964-2046, :1662-1737): when
 * enabled, every kernel launch of the forward calls is bracketed by two HIP
 * events on its own stream.  qe_moe_profile_read sums the elapsed time and
 * launch count per kernel id (arrays of at least QE_MOE_NPROF entries), then
 * clears the record; qe_moe_profile_name names an id. */
#define QE_MOE_NPROF 11
int qe_moe_profile(qe_moe_ctx *ctx, int enable);
int qe_moe_profile_read(qe_moe_ctx *ctx, double *ms, int *launches, int n);
const char *qe_moe_profile_name(int id);

/* Load the MoE tensors of pack layers pack_first .. pack_first + n_layers - 1
 * from a weight pack (layout engine/pack.h:45-54) into context layers
 * first_layer .. first_layer + n_layers - 1: blk.N.experts (256 NL4 blobs),
 * post_norm, router + sh_gate (F32), sh_gate_proj + sh_up and sh_down (Q8).
 * Replaces Pack (engine/qe.cpp:50-71) and the MoE part of Engine::Engine's
 * uploads (engine/qe.cpp:1051-1057, :1172-1194).  A missing tensor, another
 * format or a size mismatch returns QE_ERR_ARG (the reference exits).
 * Synchronous: returns once the copies are done. */
int qe_moe_load_pack(qe_moe_ctx *ctx, const char *path, int pack_first, int first_layer, int n_layers, void *stream);

/* IQ4_NL conversion (the converter, engine/qconv.cpp).  Source tensors are
 * ggml tensors in device memory, contiguous 32-element blocks of one of these
 * ggml type ids (ggml.h enum ggml_type): F32 (128 B), F16 and BF16 (64 B),
 * Q8_0 (34 B: fp16 scale d, then 32 int8; value = d * q).  Every block is
 * quantized by ggml's IQ4_NL quantizer as the reference calls it
 * (ggml_quantize_chunk(GGML_TYPE_IQ4_NL, ..., imatrix = NULL)), to an fp16
 * scale and 16 code bytes in the NL4 row layout. */
#define QE_SRC_F32 0
#define QE_SRC_F16 1
#define QE_SRC_Q8_0 8
#define QE_SRC_BF16 30

/* `rows` rows of `cols` source weights -> NL4 rows of cols/2 code bytes then
 * cols/32 fp16 scales, contiguous in `dst`, on the calling thread's current
 * device (no context).  cols must be a multiple of 256,
 * src and dst 16-byte aligned, rows * cols / 32 < 2^31.  Replaces quant_row
 * (F_NL4) over dequant_rows' output (engine/qconv.cpp:91-98, :17-43). */
int qe_moe_nl4_quantize_rows(const void *src, int src_type, int64_t rows, int cols, void *dst, void *stream);

/* Convert one layer's routed experts into the arena of `layer`: gate and up
 * are blk.N.ffn_gate_exps / ffn_up_exps ([256][512][2048] weights), down is
 * blk.N.ffn_down_exps ([256][2048][512]), all of src_type.  Expert e's blob
 * gets its 512 gate rows, 512 up rows and 2048 down rows, which is the pack's
 * blk.N.experts entry.  Replaces convert_experts (engine/qconv.cpp:202-227). */
int qe_moe_convert_experts(qe_moe_ctx *ctx, int layer, const void *gate, const void *up, const void *down,
                           int src_type, void *stream);

/* Device pointer of a layer's expert arena (256 blobs), for callers that fill
 * it in place. */
int qe_moe_arena_ptr(qe_moe_ctx *ctx, int layer, void **dev);

/* Fill a layer (experts + dense weights) on the device from the seeded
 * synthetic generator; bias (host fp32[256], NULL = none) is stored as the
 * router bias.  Benchmark/test set-up, no reference counterpart: the
 * reference loads real weights from a pack. */
int qe_moe_synth_layer(qe_moe_ctx *ctx, int layer, uint64_t seed, const float *bias, void *stream);
/* Fill n fp32 activations N(0,1) of activation set `inst` on the device. */
int qe_moe_synth_x(uint64_t seed, int inst, float *dev_out, int64_t n, void *stream);
/* The benchmark router bias of a layer (host fp32[256]): b_e = -s * ln(rank_e)
 * over a seeded permutation of the ranks 1..256, i.e. log Zipf(s) popularity
 * (3, 4).  Host only, no device work. */
int qe_moe_synth_zipf_bias(uint64_t seed, int layer, double s, float *out);

/* Poll timeouts.  The T <= 8 path synchronises workgroups through bounded
 * polls, and so do the down workgroups of the fused prefill launch (32..4095
 * tokens) waiting for their item's gate/up workgroups; a wait that gives up (a
 * hung or starved peer) lets the launch finish with invalid outputs and
 * records it in a host-visible word.
 * The next call that looks reports each such launch once as QE_ERR_STATE:
 * every forward entry point checks at entry (without synchronising, so a
 * launch still running is reported by a later call), and qe_moe_get_routing,
 * qe_moe_get_logits and qe_moe_check after synchronising `stream`.  The
 * reference has no counterpart (its queue waits cannot fail). */
int qe_moe_check(qe_moe_ctx *ctx, void *stream);

/* Test hooks, no reference counterpart.  qe_moe_debug_set_epoch writes the
 * decode launch counter (its low 16 bits tag the exchanged words), so a test
 * can run launches across the counter's wrap; qe_moe_debug_set_spin_cap sets
 * the reads an exchange poll (decode) or a down workgroup's wait for its item
 * (the fused prefill launch, 32..4095 tokens) makes before giving up (0 = the
 * default), so a test can force a timeout without a stalled kernel. */
int qe_moe_debug_set_epoch(qe_moe_ctx *ctx, uint32_t epoch, void *stream);
int qe_moe_debug_set_spin_cap(qe_moe_ctx *ctx, int cap);
/* Test hook, no reference counterpart: the fused prefill launch's down
 * workgroups wait for `extra` more gate/up workgroups than their item has (0 =
 * as in use), so that every such wait gives up after the spin cap. */
int qe_moe_debug_fused_wait_extra(qe_moe_ctx *ctx, int extra);

const char *qe_moe_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
