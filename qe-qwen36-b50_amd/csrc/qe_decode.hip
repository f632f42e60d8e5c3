// Persistent decode kernel: T <= 8 tokens through n_layers MoE layers in ONE
// launch (the MoE sections of Engine::decode, engine/qe.cpp:2466-2572, and
// decode_multi<NT>, :1653-1737, looped over the layers as at :2241).
//
// Its workgroups wait for each other, so all of them must be resident at once:
// one per CU (the LDS use admits no second), at most as many as there are
// CUs.  A plain launch of that grid on an otherwise idle device puts every
// workgroup on its own CU; hipLaunchCooperativeKernel guarantees the same but
// measured 18 us more per launch (37 against 19 us for one layer).  Should
// another kernel hold CUs, the late workgroups start when it ends; the polls
// are bounded either way, and a timeout is reported to the caller.
//
// Why persistent: on MI355X every kernel launch costs ~4.5 us of fixed
// duration (dispatch over 8 XCDs + end-of-kernel L2 write-back), while one
// B=1 layer moves 19.6 MB = 2.5 us at 8 TB/s.
//
// One 1024-thread workgroup (16 waves) per CU.  Per layer:
//   R  x -> RMSNorm -> int8 x (every workgroup, redundantly); router rows and
//      shared gate|up row pairs, one wave per row task      -> logits, silu(g)*u
//   G  top-8 + dispatch (every workgroup, redundantly); routed gate/up + SwiGLU
//      on units of 16 (T = 1) or 32 (T > 1) hidden rows of one expert, spread
//      over all workgroups                                    -> h
//   D  routed down (rows prefetched into registers during G), shared down, combine,
//      residual, 8 output rows per workgroup                  -> next x
// Every value crossing workgroups is one 64-bit agent-scope store {value, tag}
// with tag = (launch epoch, layer, stage), so a reader verifies what it reads.
// Agent-scope relaxed atomics compile to sc1 accesses, coherent across the
// XCDs' separate L2s without write-back fences.  Consumers poll the data
// itself: the logits and shared activations word by word; for the all-gathers
// of x and h, one word per producer first (the last it writes), then all of it
// once with the tags verified (a word not there yet is re-read).
// Every exchanged buffer exists in REP copies: producers write all of them, a
// workgroup reads copy blockIdx % REP, so ~64 workgroups poll any one cache
// line instead of all 256 (the shared lines otherwise queue the polls at
// their memory channel: ~5 us per exchange against a 0.6 us one-way
// store->load latency measured between two workgroups).
// Buffer reuse needs no counters; the data flow orders it.  A workgroup
// rewrites a buffer for layer l+1 only after reading all of x of layer l, and
// every workgroup wrote its rows of x after its reads of layer l's logits, h
// and shared activations, which those rows depend on (x itself alternates
// between two buffers).  Weights a stage needs that do not depend on the data
// being waited for are loaded before the wait.
#include "qe_kernels.h"

#include <atomic>
#include <mutex>

#define LD_A(p) __hip_atomic_load((p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
#define ST_A(p, v) __hip_atomic_store((p), (v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
#define ADD_A(p, v) __hip_atomic_fetch_add((p), (v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)

#define DEC_T QE_SMALL_T
#define NWV 16            /* waves per workgroup */
#define NTH (NWV * 64)
#define SYNC_EPOCH 0
#define SYNC_EXIT 32
#define REP QE_DEC_REP      /* copies of every exchanged buffer and counter */
#define DEC_MIN_GRID 64   /* D row groups per workgroup stay <= 4 */
#define N_RTASK (QE_ROUTER_ROWS + QE_FF_SH) /* router rows, then shared (gate, up) row pairs */

// LDS layout (bytes).  Rows read one 32-element chunk per lane are padded to
// 33 words per chunk (or stored chunk-transposed) so a wave's reads hit 64
// distinct banks instead of one.
#define DEC_XSTR (QE_D + 32)                        /* floats per token in s_xn */
QE_DEV int xpos(int e) { return (e & 31) * 65 + (e >> 5); } // raw x element e of a token in s_xn
#define L_U 0                                       // union, by stage:
#define L_XN L_U                                    //   R: f32 [T][DEC_XSTR]: raw x, then xn, element e at xpos(e)
#define L_GU L_U                                    //   G: f32 [64 rows][8 pairs] gate/up dots of a unit
#define L_HQ (L_U + 64 * 8 * 4)                     //   D: int8 [T*8][512] quantised h
#define L_HS (L_HQ + DEC_T * 8 * QE_FF_EXP)         //   D: f32 [T*8][16] its block scales
#define L_Y (L_HS + DEC_T * 8 * 16 * 4)             //   D: f32 [8 rows][2 halves][T] routed partials
#define L_YG (L_Y + 8 * 2 * DEC_T * 4)              //   D, T > 1: f32 [16 waves][4 lane groups][T] their running sums
#define L_U_END (L_U + DEC_T * DEC_XSTR * 4)
#define L_XQ L_U_END                                // int8 [T][2048]   quantised xn
#define L_XS (L_XQ + DEC_T * QE_D)                  // f32 [T][64]      its block scales
#define L_HSH (L_XS + DEC_T * 64 * 4)               // f32 [T][512]     shared-expert silu(g)*u
#define L_RES (L_HSH + DEC_T * QE_FF_SH * 4)        // f32 [T][32]      raw x of this workgroup's D rows
#define L_RW (L_RES + DEC_T * 32 * 4)               // [4 waves][8 KB] prefetched weights of the first row task
#define L_PN (L_RW + 4 * 8192)                      // f32 [32][65] post_norm, element e at (e / 64) * 65 + e % 64
#define L_ITEMS (L_PN + 32 * 65 * 4)                // int4 [64]
#define L_PAIRS (L_ITEMS + 64 * 16)                 // int [64]
#define L_IDS (L_PAIRS + 64 * 4)                    // int [64]
#define L_WTS (L_IDS + 64 * 4)                      // f32 [64]
#define L_SHG (L_WTS + 64 * 4)                      // f32 [8]
#define L_MISC (L_SHG + 8 * 4)                      // int [16]
#define L_INV (L_MISC + 16 * 4)                     // f32 [8]          1 / rms of each token
#define L_SD (L_INV + 8 * 4)                        // f32 [4][8][T]    shared-expert output of the D rows
#define L_GX (L_SD + 4 * 8 * DEC_T * 4)            // f32 [T][8] the 8 output rows of a group, per token
#define L_TK (L_GX + DEC_T * 8 * 4)            // top-8 scratch: T = 1: u64 [256] survivor order keys, f32 logit 256;
                                                    //   T > 1: u64 [8][64] survivor keys per token
#define L_LG (L_TK + 512 * 8 + 16)                   // f32 [T][257] the last layer's logits (routing sink)
#define L_IORD (L_LG + DEC_T * QE_ROUTER_ROWS * 4)   // int [64] T > 1: items in unit deal order
#define L_TKF (L_IORD + 64 * 4)                      // u32 [256] T = 1: a survivor's ordered logit by tie key
#define L_TOTAL (L_TKF + 256 * 4)
static_assert(L_YG + NWV * 4 * DEC_T * 4 <= L_U_END, "D-stage LDS must fit in the union");
static_assert(64 * 8 * 4 <= L_HQ - L_U, "G-stage LDS must fit in front of the D buffers");
static_assert(L_TOTAL <= 160 * 1024, "LDS budget of one workgroup per CU");

// exchange buffer offsets (u64 words, {value or payload, tag})
#define EX_X 0                                      // 2 x [T][2048] f32
#define EX_L (EX_X + 2 * DEC_T * QE_D)              // [T][257] f32 logits
#define EX_HSH (EX_L + DEC_T * QE_ROUTER_ROWS)      // [T][512] f32 shared silu(g)*u
#define EX_HQ (EX_HSH + DEC_T * QE_FF_SH)           // [T*8][16][9]: 8 x int8x4, 1 x f32 scale
#define EX_HF (EX_HQ + DEC_T * 8 * 16 * 9)          // [8][512] f32 h (T = 1)
#define EX_XS (EX_HF + 8 * QE_FF_EXP)               // 2 x [T][256] f32 sum-of-squares partial of each 8-row group of x
#define EX_TOTAL (EX_XS + 2 * DEC_T * 256)          // one replica
static_assert(REP * EX_TOTAL == QE_DECODE_EX_WORDS, "exchange size must match the allocation");
static_assert(SYNC_EXIT < QE_DECODE_SYNC_WORDS, "sync words must match the allocation");

QE_DEV uint64_t pack_tv(float v, unsigned tag) { return ((uint64_t)tag << 32) | __float_as_uint(v); }
QE_DEV float tv_val(uint64_t w) { return __uint_as_float((unsigned)w); }

// Bounded polling: after pc.cap failed reads a poll gives up, records the
// launch in the host-visible error word (system scope: the host reads it
// without synchronising the stream) and goes on with what it read, so every
// wave still reaches the end of the kernel.  A wave whose poll gave up makes
// every later poll of the launch with a cap of QE_DECODE_SPIN_CAP_LATE reads:
// the launch is already invalid, and it should end soon rather than wait the
// full cap once per poll (tens of minutes over 40 layers).
struct PollCtl {
    unsigned *err;  // host-mapped word: 0, or 1 + the epoch of a launch whose poll timed out
    int cap;        // reads a poll makes before it gives up (per wave; lowered after a timeout)
    unsigned val;   // what this launch records
};
QE_DEV void poll_timeout(PollCtl &pc) {
    __hip_atomic_store(pc.err, pc.val, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    pc.cap = pc.cap < QE_DECODE_SPIN_CAP_LATE ? pc.cap : QE_DECODE_SPIN_CAP_LATE;
}

// Read N tagged words w[i] = src[i * stride] until every one carries `tag`
// (wave-uniform retry, at most pc.cap reads).  Inactive lanes read nothing.
// One read in flight per retry: measured against two, four and six staggered
// reads per poller, the extra polling traffic delayed the producers' stores
// more than it shortened detection (1,680 vs 1,620 / 1,551 / 1,494 tokens/s).
template <int N>
QE_DEV void read_tv(const uint64_t *src, int stride, unsigned tag, uint64_t w[N], bool act, PollCtl &pc) {
    for (int spins = 0;; ++spins) {
        unsigned bad = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            w[i] = act ? LD_A((uint64_t *)src + (size_t)i * stride) : ((uint64_t)tag << 32);
            bad |= (unsigned)(w[i] >> 32) ^ tag;
        }
        if (__all(bad == 0)) break;
        if (spins + 1 >= pc.cap) { poll_timeout(pc); break; }
        __builtin_amdgcn_s_sleep(1);
    }
}

// The same poll for N = 2 M consecutive words (16-byte aligned), read two per
// 16-byte load: each word carries its own tag, and an aligned 8-byte word is
// never torn, so a load that catches one half written and the other not simply
// polls again.  Half the requests of M pairs of 8-byte polls.
typedef unsigned qe_dec_u32x4 __attribute__((ext_vector_type(4)));
template <int M>
QE_DEV void read_tv_pairs(const uint64_t *src, unsigned tag, uint64_t w[2 * M], PollCtl &pc) {
    for (int spins = 0;; ++spins) {
        unsigned bad = 0;
        qe_dec_u32x4 v[M];
#pragma unroll
        for (int i = 0; i < M; ++i) asm volatile("global_load_dwordx4 %0, %1, off sc1" : "=v"(v[i]) : "v"(src + 2 * i) : "memory");
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < M; ++i) {
            w[2 * i] = ((uint64_t)v[i].y << 32) | v[i].x;
            w[2 * i + 1] = ((uint64_t)v[i].w << 32) | v[i].z;
            bad |= (v[i].y ^ tag) | (v[i].w ^ tag);
        }
        if (__all(bad == 0)) break;
        if (spins + 1 >= pc.cap) { poll_timeout(pc); break; }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Gate/up rows of one unit: this lane's NB blocks of its row (blocks c + LPR i,
// LPR = 64 / NB lanes per row), dotted with the int8 x of every pair of the item;
// the row total lands in s_gu[row_in_unit * 8 + pair].
// after_loads() runs once the row's loads are issued (other loads can queue
// behind them there without delaying this row).
template <int NB, typename F>
QE_DEV void unit_rows(const uint8_t *row, int c, int row_in_unit, const int4 it, const int *s_pairs,
                      const int8_t *s_xq, const float *s_xs, float *s_gu, F &&after_loads) {
    constexpr int LPR = 64 / NB;
    uint4 q[NB];
    uint16_t dwr[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int b = c + LPR * i;
        q[i] = *(const uint4 *)(row + b * 16);
        dwr[i] = ((const uint16_t *)(row + QE_D / 2))[b];
    }
    after_loads();
    float dw[NB];
#pragma unroll
    for (int i = 0; i < NB; ++i) dw[i] = f16_bits_to_f32(dwr[i]);
    for (int jp = 0; jp < it.z; ++jp) {
        const int t = s_pairs[it.y + jp] / QE_K_USED;
        const int8_t *xq = s_xq + t * QE_D;
        const float *xs = s_xs + t * 64;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < NB; ++i) {
            const int b = c + LPR * i;
            const nl4_blk w = nl4_decode_block<NB == 2>(q[i]); // decoded per pair: few registers, T > 1 only repeats
            const uint4 x0 = *(const uint4 *)(xq + b * 32), x1 = *(const uint4 *)(xq + b * 32 + 16);
            acc = fmaf(dw[i] * xs[b], (float)nl4_block_dot(w, x0, x1), acc);
        }
        static_assert(LPR == 16 || LPR == 32 || LPR == 64, "row reduction over 16, 32 or 64 lanes");
        acc = sum16(acc);
        if (LPR >= 32) acc = add_rows16(acc);
        if (LPR == 64) acc = add_rows32(acc);
        if (c == 0) s_gu[row_in_unit * 8 + jp] = acc;
    }
}

// Chunk `lane` (elements 32 lane .. 32 lane + 31) of a token's x in LDS, every
// read issued before any is used.  Left to itself the scheduler streams the
// reads into an fma chain two at a time, each pair waiting for the last:
// sixteen LDS round trips in series.
QE_DEV void lds_chunk32(const float *xt, int lane, float (&c)[32]) {
#pragma unroll
    for (int i = 0; i < 32; ++i) c[i] = xt[i * 65 + lane];
    __builtin_amdgcn_sched_barrier(0);
}

// Q8_0 quantisation of 8 consecutive elements held by one lane, four lanes
// (xor 1, 2 neighbours) per 32-block: block maximum, scale, int8 values; the
// scale is stored where xs is not null (one lane of the four).
QE_DEV void quant8_block4(const float (&v)[8], int8_t *xq, float *xs) {
    float am = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) am = fmaxf(am, fabsf(v[i]));
    am = fmaxf(am, dpp_f<QE_DPP_XOR1>(am));
    am = fmaxf(am, dpp_f<QE_DPP_XOR2>(am));
    float dq;
    const float id = quant_scale_inv(am, dq);
    unsigned q[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i >> 2] |= (unsigned)(uint8_t)quant_one(v[i], id) << (8 * (i & 3));
    *(uint2 *)xq = make_uint2(q[0], q[1]);
    if (xs) *xs = dq;
}

// TM = 1: the single-token kernel (B = 1 decode); TM = 8: any T <= 8.
template <int TM, bool EXN>
__global__ __launch_bounds__(NTH) void k_decode(QeDecodeArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    float *s_xn = (float *)(lds + L_XN);
    float *s_pn = (float *)(lds + L_PN);
    float *s_inv = (float *)(lds + L_INV);
    float *s_sd = (float *)(lds + L_SD);
    float *s_gu = (float *)(lds + L_GU);
    int8_t *s_hq = (int8_t *)(lds + L_HQ);
    float *s_hs = (float *)(lds + L_HS);
    float *s_y = (float *)(lds + L_Y);
    int8_t *s_xq = (int8_t *)(lds + L_XQ);
    float *s_xs = (float *)(lds + L_XS);
    float *s_hsh = (float *)(lds + L_HSH);
    float *s_res = (float *)(lds + L_RES);
    int4 *s_items = (int4 *)(lds + L_ITEMS);
    int *s_pairs = (int *)(lds + L_PAIRS);
    int *s_ids = (int *)(lds + L_IDS);
    float *s_wts = (float *)(lds + L_WTS);
    float *s_shg = (float *)(lds + L_SHG);
    int *s_misc = (int *)(lds + L_MISC);

    const int T = TM == 1 ? 1 : a.T, np = T * QE_K_USED;
    const int d_iters = (QE_D / 8 + gridDim.x - 1) / gridDim.x; // D row groups of 8 per workgroup
    if (threadIdx.x == 0) {
        s_misc[1] = (int)LD_A(a.sync + SYNC_EPOCH);
        s_misc[3] = 0; // T = 1: tag of the layer whose 1/rms is in s_inv (tags are never 0)
    }
    __syncthreads();
    const unsigned epoch = (unsigned)s_misc[1];
    PollCtl pc{a.err, a.spin_cap, 1u + (epoch & 0x7fffffffu)};
    uint64_t *EX = a.ex;                                   // replica 0 (writes go to all REP)
    const uint64_t *EXr = a.ex + (size_t)(blockIdx.x % REP) * EX_TOTAL; // the copy this workgroup reads
    constexpr bool mode16 = TM == 1; // 16-row units, fp32 h (one token: 8 items x 32 units fill the grid)
    const int rb0 = blockIdx.x * 8;

    for (int li = 0; li < a.n_layers; ++li) {
        // Thread indices re-derived per layer through an opaque copy: addresses built
        // from them stay inside the loop instead of being hoisted out and spilled.
        int tid = threadIdx.x;
        asm volatile("" : "+v"(tid));
        const int lane = tid & 63, wv = tid >> 6, l16 = lane & 15;
        // D (shared down rows, and the T > 1 routed down): wave = (row rr of the group
        // of 8, half); items u = half + 2 s, slot s = 4 k + isub.  The T = 1 routed
        // down has its own layout (wave = item wv / 2, half wv % 2).
        const int rr = wv >> 1, half = wv & 1, isub = lane >> 4;
        const int l = a.first_layer + li;
        const bool last = li == a.n_layers - 1;
        const unsigned tagR = epoch * 65536u + (unsigned)li * 4u + 1u; // logits, shared h
        const unsigned tagG = tagR + 1u;                               // routed h
        const unsigned tagD = tagR + 2u;                               // x of the next layer
        const unsigned tagIn = tagR - 2u;                              // x of this layer (li > 0)
        const uint64_t *src_x = EXr + EX_X + (size_t)((li - 1) & 1) * DEC_T * QE_D;
        uint64_t *dst_x = EX + EX_X + (size_t)(li & 1) * DEC_T * QE_D;
        const uint64_t *src_xs = EXr + EX_XS + (size_t)((li - 1) & 1) * DEC_T * 256;
        uint64_t *dst_xs = EX + EX_XS + (size_t)(li & 1) * DEC_T * 256;
        const uint8_t *arena = a.arena + (size_t)l * QE_LAYER_EXPERT_BYTES;
        const float *router = a.router + (size_t)l * QE_ROUTER_ROWS * QE_D;
        const float *bias = a.bias_on[l] ? a.bias + (size_t)l * QE_N_EXPERT : nullptr;
        const uint8_t *sh_gu = a.sh_gu + (size_t)l * QE_SH_GU_BYTES;
        const uint8_t *sh_dn = a.sh_dn + (size_t)l * QE_SH_DN_BYTES;
        const float *pnorm = a.norm ? a.post_norm + (size_t)l * QE_D : nullptr;

        // ================= R: x, norm, router rows + shared (gate, up) pairs =================
        // this wave's first row task into registers before waiting for x
        // The first row task of waves 0..3 is copied into LDS before waiting for x
        // (global->LDS, no registers held): a router row as 2048 fp32, or a shared
        // (gate, up) pair as 2 x 2048 int8 + 2 x 64 scales, one u16 per dword.
        // T = 1: wave 0 takes no row task; it polls the logits next, and a poll
        // issued after a store of its own would wait for that store's
        // acknowledgement as well (vmcnt counts both).
        constexpr int TW0 = TM == 1 ? 1 : 0;  // first wave with row tasks
        const int task0 = wv < TW0 ? N_RTASK : blockIdx.x + (int)gridDim.x * (wv - TW0);
        uint8_t *rw_lds = lds + L_RW + ((wv - TW0) & 3) * 8192;
        const bool rw_pref = wv >= TW0 && wv < TW0 + 4 && task0 < N_RTASK;
        if (rw_pref) {
            // Lane i's 16 bytes land at dst + 16 i; the source is the i-th lane chunk's
            // k-th 16 bytes, so the dot (lane = chunk) reads dst + 16 lane: no bank conflicts.
            auto dma16 = [&](const uint8_t *src, uint8_t *dst) {
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                                 (__attribute__((address_space(3))) void *)dst, 16, 0, 0);
            };
            if (task0 < QE_ROUTER_ROWS) { // chunk = 128 B of fp32
                const uint8_t *row = (const uint8_t *)(router + (size_t)task0 * QE_D);
#pragma unroll
                for (int k = 0; k < 8; ++k) dma16(row + lane * 128 + k * 16, rw_lds + k * 1024);
            } else { // chunk = 32 B of int8 per matrix
                const int j = task0 - QE_ROUTER_ROWS;
                const uint8_t *rg = sh_gu + (size_t)j * QE_SH_GU_ROW_BYTES, *ru = sh_gu + (size_t)(QE_FF_SH + j) * QE_SH_GU_ROW_BYTES;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    dma16(rg + lane * 32 + k * 16, rw_lds + k * 1024);
                    dma16(ru + lane * 32 + k * 16, rw_lds + 2048 + k * 1024);
                }
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(rg + QE_D + lane * 2),
                                                 (__attribute__((address_space(3))) void *)(rw_lds + 4096), 2, 0, 0);
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(ru + QE_D + lane * 2),
                                                 (__attribute__((address_space(3))) void *)(rw_lds + 4096 + 256), 2, 0, 0);
            }
        }
        // post_norm -> LDS, 64-element rows padded to 65 words (one dword per lane);
        // T = 1 after the first layer: by wave 0, whose partials poll waits for it
        // before it signals 1/rms to the threads that scale x as it arrives
        if (pnorm && wv == (TM == 1 && li > 0 ? 0 : 4)) {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(pnorm + i * 64 + lane),
                                                 (__attribute__((address_space(3))) void *)(s_pn + i * 65), 4, 0, 0);
        }
        // x of a layer li > 0: wave t first polls token t's 256 group partials of
        // the sum of squares (published with x, one word per 8-row group), which
        // give 1/rms at once (canonical order: lane l holds groups 4l..4l+3); then
        // the whole workgroup reads x, each thread polling its own words (at T = 1
        // and scaling them: no pass of its own, one barrier fewer).
        if (li > 0 && wv < T) {
            const int t = wv;
            uint64_t w[4];
            read_tv_pairs<2>(src_xs + t * 256 + 4 * lane, tagIn, w, pc);
            const float ss = wave_sum_canon((tv_val(w[0]) + tv_val(w[1])) + (tv_val(w[2]) + tv_val(w[3])));
            if (lane == 0) s_inv[t] = 1.0f / sqrtf(ss / (float)QE_D + QE_RMS_EPS);
            if (TM == 1) {
                // 1/rms and post_norm are in place: post_norm came by global->LDS loads of
                // this wave, which complete into LDS only as vmcnt drains, and a
                // workgroup-scope release does not wait for vmcnt
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                if (lane == 0) __hip_atomic_store(&s_misc[3], (int)tagIn, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
        // raw x of all tokens -> LDS (natural layout, token stride 2048; T*2048 = 2 T NTH)
        if (li == 0) {
            if constexpr (TM == 1) { // both loads issued before either is stored
                const float x0 = a.x_in[tid], x1 = a.x_in[tid + NTH];
                s_xn[xpos(tid)] = x0;
                s_xn[xpos(tid + NTH)] = x1;
            } else { // loads issued four at a time before their stores
                for (int k0 = 0; k0 < 2 * T; k0 += 4) {
                    float xv[4];
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        if (k0 + k < 2 * T) xv[k] = a.x_in[tid + (k0 + k) * NTH];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const int i = tid + (k0 + k) * NTH;
                        if (k0 + k < 2 * T) s_xn[(i >> 11) * DEC_XSTR + xpos(i & 2047)] = xv[k];
                    }
                }
            }
        } else if (TM == 1 || T <= 2) {
            for (int i0 = 0; i0 < T * QE_D; i0 += 2 * NTH) {
                uint64_t w[2];
                read_tv_pairs<1>(src_x + i0 + 2 * tid, tagIn, w, pc);
                const int e0 = i0 + 2 * tid, e1 = e0 + 1;
                float x0 = tv_val(w[0]), x1 = tv_val(w[1]);
                if (TM == 1 && pnorm) { // scaled as it arrives, once wave 0 has 1/rms
                    while (__hip_atomic_load(&s_misc[3], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) != (int)tagIn) {
                    }
                    const float inv = s_inv[0];
                    x0 = (x0 * inv) * s_pn[(e0 >> 6) * 65 + (e0 & 63)];
                    x1 = (x1 * inv) * s_pn[(e1 >> 6) * 65 + (e1 & 63)];
                }
                s_xn[(e0 >> 11) * DEC_XSTR + xpos(e0 & 2047)] = x0;
                s_xn[(e1 >> 11) * DEC_XSTR + xpos(e1 & 2047)] = x1;
            }
        } else {
            // up to 16 words per thread: 8 polled together per round trip (T = 8: two)
            for (int i0 = 0; i0 < T * QE_D; i0 += 8 * NTH) {
                const int nw = (T * QE_D - i0) / NTH; // words left per thread: even (T * 2048 = 2 T NTH)
                uint64_t w[8];
                if (nw >= 8) {
                    read_tv<8>(src_x + i0 + tid, NTH, tagIn, w, true, pc);
                } else if (nw >= 4) {
                    read_tv<4>(src_x + i0 + tid, NTH, tagIn, w, true, pc);
                    if (nw == 6) read_tv<2>(src_x + i0 + 4 * NTH + tid, NTH, tagIn, w + 4, true, pc);
                } else {
                    read_tv<2>(src_x + i0 + tid, NTH, tagIn, w, true, pc);
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int e = i0 + tid + i * NTH;
                    if (i < nw) s_xn[(e >> 11) * DEC_XSTR + xpos(e & 2047)] = tv_val(w[i]);
                }
            }
        }
        __syncthreads();
        // First layer of the launch (x from the caller, no partials): wave t forms
        // token t's sum of squares in the canonical order (lane l holds elements
        // [32l, 32l+32)).
        if (li == 0 && pnorm && wv < T) {
            const int t = wv;
            const float *xt = s_xn + t * DEC_XSTR;
            float c[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) c[i] = xt[i * 65 + lane];
            const float ss = wave_sum_canon(sumsq_lane32(c));
            if (lane == 0) s_inv[t] = 1.0f / sqrtf(ss / (float)QE_D + QE_RMS_EPS);
        }
        if (li == 0) __syncthreads(); // later layers had 1/rms before the x read
        // RMSNorm in place.  A thread that scales elements of this workgroup's D
        // rows keeps their raw values first (the residual): no other thread
        // writes them.
        //   T = 1: the first layer of a launch, one element per thread and step;
        //          later layers scaled x as it arrived and carry the residual from
        //          the previous layer's combine.  The row tasks below need only
        //          this fp32 xn, and its int8 quantisation for the routed units
        //          is done after the barrier by wave 0, which has no row task.
        //   T > 1: 8 elements per thread, scaled and quantised (4 lanes per
        //          32-block) in one pass.
        if constexpr (TM == 1) {
            if (li == 0) {
                for (int e = tid; e < QE_D; e += NTH) {
                    float *px = s_xn + xpos(e);
                    float v = *px;
                    if (a.residual)
                        for (int m = 0; m < d_iters; ++m)
                            if ((e >> 3) == (int)blockIdx.x + m * (int)gridDim.x) s_res[m * 8 + (e & 7)] = v;
                    if (pnorm) {
                        v = (v * s_inv[0]) * s_pn[(e >> 6) * 65 + (e & 63)];
                        *px = v;
                    }
                    if (last && blockIdx.x == 0 && a.xn_out) a.xn_out[e] = v;
                }
                __syncthreads();
            } else if (last && blockIdx.x == 0 && a.xn_out && wv == NWV - 1) {
                // (a wave without a row task: a store of wave 0's own would hold up its logits poll)
                for (int e = lane; e < QE_D; e += 64) a.xn_out[e] = s_xn[xpos(e)];
            }
        } else {
            for (int w = tid; w < T * 256; w += NTH) {
                const int t = w >> 8, e = 8 * (w & 255);
                float *xt = s_xn + t * DEC_XSTR;
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = xt[xpos(e + i)];
                if (a.residual)
                    for (int m = 0; m < d_iters; ++m)
                        if ((w & 255) == (int)blockIdx.x + m * (int)gridDim.x) {
#pragma unroll
                            for (int i = 0; i < 8; ++i) s_res[t * 32 + m * 8 + i] = v[i];
                        }
                if (pnorm) {
                    const float inv = s_inv[t];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = (v[i] * inv) * s_pn[(e >> 6) * 65 + (e & 63) + i];
                }
#pragma unroll
                for (int i = 0; i < 8; ++i) xt[xpos(e + i)] = v[i];
                quant8_block4(v, s_xq + t * QE_D + e, (w & 3) == 0 ? s_xs + t * 64 + (e >> 5) : nullptr);
                if (last && blockIdx.x == 0 && a.xn_out) {
                    float4 *o = (float4 *)(a.xn_out + (size_t)t * QE_D + e);
                    o[0] = make_float4(v[0], v[1], v[2], v[3]);
                    o[1] = make_float4(v[4], v[5], v[6], v[7]);
                }
            }
            __syncthreads();
        }
        for (int task = task0; task < N_RTASK; task += (int)gridDim.x * (NWV - TW0)) {
            const bool in_lds = rw_pref && task == task0;
            if (task < QE_ROUTER_ROWS) {
                const bool add_bias = bias && task < QE_N_EXPERT;
                const float b = add_bias ? bias[task] : 0.f;
                float wr[32];
                if (in_lds) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) *(float4 *)(wr + 4 * i) = *(const float4 *)(rw_lds + i * 1024 + lane * 16);
                } else {
                    load32(router + (size_t)task * QE_D + lane * 32, wr);
                }
                for (int t = 0; t < T; ++t) {
                    float xv[32];
                    if constexpr (TM == 1) {
                        lds_chunk32(s_xn, lane, xv);
                    } else {
#pragma unroll
                        for (int i = 0; i < 32; ++i) xv[i] = s_xn[t * DEC_XSTR + i * 65 + lane];
                    }
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) acc = fmaf(wr[i], xv[i], acc);
                    acc = wave_sum_canon(acc);
                    if (lane < REP) ST_A(EX + lane * EX_TOTAL + EX_L + t * QE_ROUTER_ROWS + task, pack_tv(add_bias ? acc + b : acc, tagR));
                }
            } else {
                const int j = task - QE_ROUTER_ROWS;
                uint4 g0, g1, u0, u1;
                float gsc, usc;
                if (in_lds) {
                    g0 = *(const uint4 *)(rw_lds + lane * 16);
                    g1 = *(const uint4 *)(rw_lds + 1024 + lane * 16);
                    u0 = *(const uint4 *)(rw_lds + 2048 + lane * 16);
                    u1 = *(const uint4 *)(rw_lds + 3072 + lane * 16);
                    gsc = f16_bits_to_f32((uint16_t)*(const unsigned *)(rw_lds + 4096 + lane * 4));
                    usc = f16_bits_to_f32((uint16_t)*(const unsigned *)(rw_lds + 4096 + 256 + lane * 4));
                } else {
                    const uint8_t *rg = sh_gu + (size_t)j * QE_SH_GU_ROW_BYTES, *ru = sh_gu + (size_t)(QE_FF_SH + j) * QE_SH_GU_ROW_BYTES;
                    g0 = ((const uint4 *)(rg + lane * 32))[0];
                    g1 = ((const uint4 *)(rg + lane * 32))[1];
                    gsc = f16_bits_to_f32(((const uint16_t *)(rg + QE_D))[lane]);
                    u0 = ((const uint4 *)(ru + lane * 32))[0];
                    u1 = ((const uint4 *)(ru + lane * 32))[1];
                    usc = f16_bits_to_f32(((const uint16_t *)(ru + QE_D))[lane]);
                }
                auto publish = [&](int t, float ag, float au) {
                    ag = wave_sum_canon(ag * gsc);
                    au = wave_sum_canon(au * usc);
                    const float hv = silu_mul(ag, au);
                    if (lane < REP) ST_A(EX + lane * EX_TOTAL + EX_HSH + t * QE_FF_SH + j, pack_tv(hv, tagR));
                };
                if constexpr (TM == 1) {
                    // one token: the weights stay packed (16 registers) and are
                    // widened in the chain, so x can sit in 32 registers
                    const uint32_t gd[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
                    const uint32_t ud[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
                    float xv[32];
                    lds_chunk32(s_xn, lane, xv);
                    float ag = 0.f, au = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        ag = fmaf((float)(int8_t)((gd[i >> 2] >> (8 * (i & 3))) & 0xff), xv[i], ag);
                        au = fmaf((float)(int8_t)((ud[i >> 2] >> (8 * (i & 3))) & 0xff), xv[i], au);
                    }
                    publish(0, ag, au);
                } else {
                    float wg[32], wu[32];
                    unpack_i8x32(g0, g1, wg);
                    unpack_i8x32(u0, u1, wu);
                    for (int t = 0; t < T; ++t) {
                        float ag = 0.f, au = 0.f;
#pragma unroll
                        for (int i = 0; i < 32; ++i) {
                            const float xv = s_xn[t * DEC_XSTR + i * 65 + lane];
                            ag = fmaf(wg[i], xv, ag);
                            au = fmaf(wu[i], xv, au);
                        }
                        publish(t, ag, au);
                    }
                }
            }
        }

        if constexpr (TM == 1) {
            // int8 quantisation of xn for the routed units (read in G, after the
            // workgroup barrier that follows the top-8), by wave 0 before it polls
            // the logits: 8 elements per lane and step, 4 lanes per 32-block
            if (wv == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) { // unrolled: the four blocks' chains overlap
                    const int w = lane + 64 * j, e = 8 * w;
                    float v[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i) v[i] = s_xn[xpos(e + i)];
                    quant8_block4(v, s_xq + e, (w & 3) == 0 ? s_xs + (e >> 5) : nullptr);
                }
            }
        }

        // ================= G: top-8, dispatch, routed gate/up =================
        if constexpr (TM == 1) {
            // Top-8 by one wave, lane l holding the logits of experts l + 64 j.  A
            // lane's maximum over its four, then over groups of 8 lanes, gives eight
            // maxima of distinct experts; the smallest of them bounds the 8th largest
            // logit from below, so the experts at or above it (about 18 of 256) hold
            // the top 8.  The survivors are put in the reference's total order (larger
            // value first, ties to the smaller (e % 16, e / 16)) by their keys {ordered
            // value, 0xffff - tie key}: up to 64 of them sorted in registers, more (many
            // equal logits) ranked by counting the keys above each; ranks 0..7 are the
            // selection in order.  The experts
            // become the items in rank order; the weights are formed later, off the
            // critical path (they are first needed in D).  (Rounds of wave maxima, or
            // the ranks counted by every thread over all 256, took 1-2 us per layer.)
            uint64_t *s_sk = (uint64_t *)(lds + L_TK);           // [256] survivors' order keys
            unsigned *s_full = (unsigned *)(lds + L_TKF);          // [256] survivors' logit keys by tie key
            float *s_lg256 = (float *)(lds + L_TK + 2048);
            if (wv == 0) {
                uint64_t w[5]; // the lane's four logits and (lane 0) logit 256, one poll loop
                for (int spins = 0;; ++spins) {
                    unsigned bad = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        w[j] = LD_A((uint64_t *)EXr + EX_L + lane + 64 * j);
                        bad |= (unsigned)(w[j] >> 32) ^ tagR;
                    }
                    w[4] = lane == 0 ? LD_A((uint64_t *)EXr + EX_L + QE_N_EXPERT) : ((uint64_t)tagR << 32);
                    bad |= (unsigned)(w[4] >> 32) ^ tagR;
                    if (__all(bad == 0)) break;
                    if (spins + 1 >= pc.cap) { poll_timeout(pc); break; }
                    __builtin_amdgcn_s_sleep(1);
                }
                unsigned v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = f2ord(tv_val(w[j]) + 0.0f);
                if (lane == 0) *s_lg256 = tv_val(w[4]);
                if (last && blockIdx.x == 0) { // kept for the routing sink
                    float *s_lgs = (float *)(lds + L_LG);
#pragma unroll
                    for (int j = 0; j < 4; ++j) s_lgs[lane + 64 * j] = tv_val(w[j]);
                    if (lane == 0) s_lgs[QE_N_EXPERT] = tv_val(w[4]);
                }
                unsigned g = umax32(umax32(v[0], v[1]), umax32(v[2], v[3]));
                g = umax32(g, dpp_ub<QE_DPP_XOR1>(g));
                g = umax32(g, dpp_ub<QE_DPP_XOR2>(g));
                g = umax32(g, dpp_ub<QE_DPP_HMIRROR>(g)); // maximum of 32 experts (8 lanes)
                g = umin32(g, dpp_ub<QE_DPP_MIRROR>(g));
                unsigned ra, rb;
                rows16(g, ra, rb);
                g = umin32(ra, rb);
                rows32(g, ra, rb);
                g = umin32(ra, rb); // the smallest of the eight
                int S = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) { // survivors numbered by (j, lane)
                    const bool sv = v[j] >= g;
                    const unsigned long long bal = __ballot(sv);
                    if (sv) {
                        const int e = lane + 64 * j, pos = S + (int)__builtin_amdgcn_mbcnt_hi((unsigned)(bal >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)bal, 0u));
                        const unsigned tk = (unsigned)((e & 15) * 16 + (e >> 4));
                        s_sk[pos] = ((uint64_t)v[j] << 32) | (0xffffu - tk);
                        s_full[tk] = v[j];
                    }
                    S += (int)__popcll(bal);
                }
                if (S <= 64) {
                    // up to 64 survivors: one per lane, sorted in registers (no LDS round
                    // trips; the 64-wide stage only when more than 32 survive); a key's low
                    // half holds 0xffff - tie key, so it names its expert
                    const uint64_t ki = lane < S ? s_sk[lane] : 0ull; // real keys are never 0
                    uint32_t khi = (uint32_t)(ki >> 32), klo = (uint32_t)ki;
                    // First on 32-bit keys {top 24 bits of the ordered value, 0xff - tie key}:
                    // their order is the exact one wherever no two of ranks 0..8 share the top
                    // 24 bits (every exact tie does), which one comparison with the next rank
                    // checks; otherwise the 64-bit keys are sorted.  (An ordered finite
                    // logit is >= 2^23, so real keys stay above the padding's 0.)
                    uint32_t k32 = (khi & 0xffffff00u) | (klo & 0xffu);
                    sort32_desc_u32(k32, lane);
                    if (S > 32) merge64_desc_u32(k32, lane);
                    const uint32_t nx = dpp_u<0x101>(k32); // row_shl:1, the next rank
                    if (!__any(lane < QE_K_USED && ((k32 ^ nx) >> 8) == 0u)) {
                        if (lane < QE_K_USED) {
                            const unsigned tk = 0xffu - (k32 & 0xffu); // (e % 16) * 16 + e / 16
                            s_items[lane] = make_int4((int)(((tk & 15u) << 4) | ((tk >> 4) & 15u)), lane, 1, 0);
                        }
                    } else {
                        sort32_desc_u64(khi, klo, lane);
                        if (S > 32) merge64_desc_u64(khi, klo, lane);
                        if (lane < QE_K_USED) {
                            const unsigned tk = 0xffffu - (klo & 0xffffu);
                            s_items[lane] = make_int4((int)(((tk & 15u) << 4) | ((tk >> 4) & 15u)), lane, 1, 0);
                        }
                    }
                } else {
                    for (int i0 = 0; i0 < S; i0 += 64) { // many equal logits: count the survivors ahead
                        const int i = i0 + lane;
                        const uint64_t ki = s_sk[i < S ? i : 0];
                        int r = 0, j = 0;
                        for (; j + 4 <= S; j += 4) {
                            const uint64_t k0 = s_sk[j], k1 = s_sk[j + 1], k2 = s_sk[j + 2], k3 = s_sk[j + 3];
                            r += (int)(k0 > ki) + (int)(k1 > ki) + (int)(k2 > ki) + (int)(k3 > ki);
                        }
                        for (; j < S; ++j) r += (int)(s_sk[j] > ki);
                        if (i < S && r < QE_K_USED) {
                            const unsigned tk = 0xffffu - ((unsigned)ki & 0xffffu);
                            s_items[r] = make_int4((int)(((tk & 15u) << 4) | ((tk >> 4) & 15u)), r, 1, 0);
                        }
                    }
                }
                if (lane < QE_K_USED) s_pairs[lane] = lane;
                if (lane == 0) s_misc[0] = QE_K_USED;
            }
        } else if (wv < T) {
            const int t = wv;
            uint64_t w[5]; // the lane's four logits and (lane 0) logit 256, one poll loop
            const uint64_t *src = EXr + EX_L + t * QE_ROUTER_ROWS;
            for (int spins = 0;; ++spins) {
                unsigned bad = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    w[j] = LD_A((uint64_t *)src + lane + 64 * j);
                    bad |= (unsigned)(w[j] >> 32) ^ tagR;
                }
                w[4] = lane == 0 ? LD_A((uint64_t *)src + QE_N_EXPERT) : ((uint64_t)tagR << 32);
                bad |= (unsigned)(w[4] >> 32) ^ tagR;
                if (__all(bad == 0)) break;
                if (spins + 1 >= pc.cap) { poll_timeout(pc); break; }
                __builtin_amdgcn_s_sleep(16); // ~0.4 us between polls: fewer reads of lines being written (4,586 -> 4,609 tokens/s at B = 8)
            }
            w[4] = __builtin_amdgcn_readfirstlane((unsigned)w[4]); // logit 256 to every lane
            float v[5];
#pragma unroll
            for (int j = 0; j < 5; ++j) v[j] = tv_val(w[j]);
            if (last && blockIdx.x == 0) { // kept for the routing sink
                float *s_lgs = (float *)(lds + L_LG) + t * QE_ROUTER_ROWS;
#pragma unroll
                for (int j = 0; j < 4; ++j) s_lgs[lane + 64 * j] = v[j];
                if (lane == 0) s_lgs[QE_N_EXPERT] = v[4];
            }
            wave_topk_sorted(v, v[4], lane, (uint64_t *)(lds + L_TK) + 64 * t, s_ids + t * QE_K_USED, s_wts + t * QE_K_USED,
                             s_shg + t);
        }
        __syncthreads();
        if (TM != 1 && wv == 0) {
            // stable counting sort of the T*8 pairs by expert (engine/qe.cpp:1965-1976):
            // slot of pair p = #pairs with a smaller expert + #earlier pairs with the same one
            // Counted by ballots over the 8 key bits, most significant first: at bit
            // b, the lanes that share my key above b but hold 0 where I hold 1 are
            // smaller; what remains after bit 0 are my peers.  (A loop over the
            // pairs reading each key from LDS took ~4 us per layer at T = 8.)
            const bool valid = lane < np;
            const int e = valid ? s_ids[lane] : 1 << 20;
            const unsigned long long below = (1ull << lane) - 1ull; // lane < 64
            unsigned long long eq = __ballot(valid);
            int lt = 0;
#pragma unroll
            for (int bit = 7; bit >= 0; --bit) {
                const int my = (e >> bit) & 1;
                const unsigned long long ones = __ballot(valid && my);
                if (my) lt += __popcll(eq & ~ones);
                eq &= my ? ones : ~ones;
            }
            const int rank = __popcll(eq & below), cnt = __popcll(eq);
            const bool first = valid && rank == 0;
            const unsigned long long fm = __ballot(first);
            // item = first-of-key lanes with a smaller key: the same walk over them
            unsigned long long feq = fm;
            int item = 0;
#pragma unroll
            for (int bit = 7; bit >= 0; --bit) {
                const int my = (e >> bit) & 1;
                const unsigned long long ones = __ballot(first && my);
                if (my) item += __popcll(feq & ~ones);
                feq &= my ? ones : ~ones;
            }
            if (lane < np) s_pairs[lt + rank] = lane;
            if (first) s_items[item] = make_int4(e, lt, cnt, 0);
            // the order units are dealt in: items with more pairs first (their
            // units cost more), so that a workgroup's second unit is a light one;
            // the same ballot walk over the 4-bit key 15 - cnt
            {
                const int ck = 15 - cnt;
                unsigned long long ceq = fm;
                int clt = 0;
#pragma unroll
                for (int bit = 3; bit >= 0; --bit) {
                    const int my = (ck >> bit) & 1;
                    const unsigned long long ones = __ballot(first && my);
                    if (my) clt += __popcll(ceq & ~ones);
                    ceq &= my ? ones : ~ones;
                }
                if (first) ((int *)(lds + L_IORD))[clt + __popcll(ceq & below)] = item;
            }
            if (lane == 0) s_misc[0] = __popcll(fm);
        }
        if (TM != 1) __syncthreads();
        const int nitems = s_misc[0];

        // Down rows of this workgroup's first D row group for the first items and
        // the wave's shared down row, loaded into registers during G (after the
        // first unit's own loads, so the unit does not wait for them).
        //   T = 1: wave (item wv / 2, half wv % 2), lane (row lane / 8, block
        //          8 half + lane % 8): the block its routed down needs first.
        //   T > 1: wave (row rr, half), item round k = 0: lane (isub, block) takes item
        //          half + 2 isub.
        uint4 dpq[1] = {make_uint4(0, 0, 0, 0)};
        unsigned dps[1] = {0u};
        uint4 dq0 = make_uint4(0, 0, 0, 0), dq1 = dq0;
        uint16_t dsc = 0;
        bool d_prefetched = false;
        auto d_prefetch = [&]() {
            if (d_prefetched) return;
            d_prefetched = true;
            if constexpr (TM == 1) {
                // wave (item wv / 2, half wv % 2), lane (row lane / 8, block 8 half + lane % 8)
                const int u = wv >> 1, b = 8 * (wv & 1) + (lane & 7);
                const uint8_t *drow = arena + (size_t)(s_items[u].x & (QE_N_EXPERT - 1)) * QE_EXPERT_BYTES +
                                      QE_EXPERT_DOWN_OFF + (size_t)(rb0 + (lane >> 3)) * QE_DN_ROW_BYTES;
                dpq[0] = *(const uint4 *)(drow + b * 16);
                dps[0] = ((const uint16_t *)(drow + QE_FF_EXP / 2))[b];
            } else if (half < nitems) { // item round k = 0 (the routed down loads each later one itself)
                int u = half + 2 * isub;
                if (u >= nitems) u = half; // a valid item; the slot is never used
                const uint8_t *drow = arena + (size_t)s_items[u].x * QE_EXPERT_BYTES + QE_EXPERT_DOWN_OFF +
                                      (size_t)(rb0 + rr) * QE_DN_ROW_BYTES;
                dpq[0] = *(const uint4 *)(drow + l16 * 16);
                dps[0] = ((const uint16_t *)(drow + QE_FF_EXP / 2))[l16];
            }
            if (half == 0) {
                const uint8_t *srow = sh_dn + (size_t)(rb0 + rr) * QE_SH_DN_ROW_BYTES;
                dq0 = ((const uint4 *)(srow + l16 * 32))[0];
                dq1 = ((const uint4 *)(srow + l16 * 32))[1];
                dsc = ((const uint16_t *)(srow + QE_FF_SH))[l16];
            }
        };

        // Units of one expert item: JU hidden rows j (gate rows j, up rows 512 + j).
        //   mode16 (T = 1): JU = 16; wave w -> h row j0 + w: its gate row in lanes
        //                   0..31, its up row in lanes 32..63, a lane holds blocks c,
        //                   c + 32.  The wave forms h = silu(g) * u and publishes it
        //                   (fp32) itself: no workgroup barrier.
        //   else:           JU = 32, 64 rows; wave w -> 4 rows, 16 lanes per row, a lane
        //                   holds blocks c + 16 i.  h quantised per 32 rows, published int8.
        const int JU = mode16 ? 16 : 32, upi = QE_FF_EXP / JU, nunits = nitems * upi;
        auto no_prefetch = []() {};
        if constexpr (TM == 1) {
            // The shared-expert activations (written in R) are read here, their
            // loads in flight with the unit's, instead of on the h wait in D; they
            // are issued behind the unit's rows, which every workgroup requests at
            // once and whose drain from HBM bounds this stage (issued first, they
            // had cost 1.6 %).
            uint64_t hsh_w = 0;
            bool hsh_issued = false;
            for (int unit = blockIdx.x; unit < nunits; unit += gridDim.x) {
                const int4 it = s_items[unit / upi];
                const int j = (unit % upi) * JU + wv, c = lane & 31;
                const uint8_t *row = arena + (size_t)(it.x & (QE_N_EXPERT - 1)) * QE_EXPERT_BYTES +
                                     (size_t)((lane >= 32 ? QE_FF_EXP : 0) + j) * QE_GU_ROW_BYTES;
                const uint4 q0 = *(const uint4 *)(row + c * 16), q1 = *(const uint4 *)(row + (c + 32) * 16);
                const uint16_t r0 = ((const uint16_t *)(row + QE_D / 2))[c], r1 = ((const uint16_t *)(row + QE_D / 2))[c + 32];
                // x blocks c, c + 32 from LDS while the rows are on their way
                const uint4 xa = *(const uint4 *)(s_xq + c * 32), xb = *(const uint4 *)(s_xq + c * 32 + 16);
                const uint4 xc = *(const uint4 *)(s_xq + (c + 32) * 32), xd = *(const uint4 *)(s_xq + (c + 32) * 32 + 16);
                const float xs0 = s_xs[c], xs1 = s_xs[c + 32];
                if (!hsh_issued) { hsh_issued = true; if (tid < QE_FF_SH) hsh_w = LD_A((uint64_t *)EXr + EX_HSH + tid); }
                __builtin_amdgcn_sched_barrier(0);
                const float d0 = f16_bits_to_f32(r0) * xs0, d1 = f16_bits_to_f32(r1) * xs1;
                float acc = d0 * (float)nl4_block_dot(nl4_decode_block<true>(q0), xa, xb);
                acc = fmaf(d1, (float)nl4_block_dot(nl4_decode_block<true>(q1), xc, xd), acc);
                acc = add_rows16(sum16(acc)); // lanes 0..31: g, lanes 32..63: u
                const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
                const float u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 32));
                const float h = silu_mul(g, u);
                const int p = s_pairs[it.y & 7];
                if (unit == (int)blockIdx.x && tid < QE_FF_SH) {
                    // consumed before the publication below: a wait for a load after
                    // a store is a wait for the store's acknowledgement too (vmcnt
                    // counts both), ~1 us for these write-through stores
                    uint64_t w1[1] = {hsh_w};
                    if ((unsigned)(w1[0] >> 32) != tagR) read_tv<1>(EXr + EX_HSH + tid, 0, tagR, w1, true, pc);
                    s_hsh[tid] = tv_val(w1[0]);
                }
                if (lane < REP) ST_A(EX + lane * EX_TOTAL + EX_HF + (size_t)p * QE_FF_EXP + j, pack_tv(h, tagG));
            }
            if ((int)blockIdx.x >= nunits && tid < QE_FF_SH) { // no unit here
                uint64_t w1[1] = {LD_A((uint64_t *)EXr + EX_HSH + tid)};
                if ((unsigned)(w1[0] >> 32) != tagR) read_tv<1>(EXr + EX_HSH + tid, 0, tagR, w1, true, pc);
                s_hsh[tid] = tv_val(w1[0]);
            }
        } else
        for (int unit = blockIdx.x; unit < nunits; unit += gridDim.x) {
            const int4 it = s_items[((const int *)(lds + L_IORD))[unit / upi]];
            const int j0 = (unit % upi) * JU;
            const bool up = wv >= 8;
            const uint8_t *base = arena + (size_t)it.x * QE_EXPERT_BYTES + (size_t)(up ? QE_FF_EXP : 0) * QE_GU_ROW_BYTES;
            if (mode16) {
                const int rw = (wv & 7) * 2 + (lane >> 5);
                unit_rows<2>(base + (size_t)(j0 + rw) * QE_GU_ROW_BYTES, lane & 31, (up ? JU : 0) + rw, it, s_pairs,
                             s_xq, s_xs, s_gu, no_prefetch);
            } else {
                const int rw = (wv & 7) * 4 + (lane >> 4);
                unit_rows<4>(base + (size_t)(j0 + rw) * QE_GU_ROW_BYTES, l16, (up ? JU : 0) + rw, it, s_pairs,
                             s_xq, s_xs, s_gu, no_prefetch);
            }
            __syncthreads();
            if (mode16) {
                if (tid < JU * it.z) { // thread (pair jp, row j)
                    const int jp = tid / JU, j = tid % JU;
                    const float h = silu_mul(s_gu[j * 8 + jp], s_gu[(JU + j) * 8 + jp]);
                    const int p = s_pairs[it.y + jp];
#pragma unroll
                    for (int r = 0; r < REP; ++r) ST_A(EX + r * EX_TOTAL + EX_HF + (size_t)p * QE_FF_EXP + j0 + j, pack_tv(h, tagG));
                }
            } else if (tid < 32 * it.z) { // thread (pair jp, row r): quantise the unit's 32 rows
                const int jp = tid >> 5, r = tid & 31;
                const float hv = silu_mul(s_gu[r * 8 + jp], s_gu[(32 + r) * 8 + jp]);
                float amax = fabsf(hv);
                amax = max32(amax);
                float d;
                const float id = quant_scale_inv(amax, d);
                const unsigned qv = (unsigned)(uint8_t)quant_one(hv, id);
                const unsigned q1 = __shfl_down(qv, 1, 64), q2 = __shfl_down(qv, 2, 64), q3 = __shfl_down(qv, 3, 64);
                const int p = s_pairs[it.y + jp];
                uint64_t *dstw = EX + EX_HQ + ((size_t)p * 16 + j0 / 32) * 9;
#pragma unroll
                for (int rp = 0; rp < REP; ++rp) {
                    if ((r & 3) == 0) ST_A(dstw + rp * EX_TOTAL + (r >> 2), ((uint64_t)tagG << 32) | (qv | (q1 << 8) | (q2 << 16) | (q3 << 24)));
                    if (r == 0) ST_A(dstw + rp * EX_TOTAL + 8, pack_tv(d, tagG));
                }
            }
            __syncthreads(); // s_gu is reused by the next unit
        }
        d_prefetch(); // workgroups without a unit
        // ================= D: routed down + shared down + combine =================
        // No counter: h is polled through its tags, every thread its own words
        // (T = 1: four, one round trip after they land).  A first poll of one
        // word per unit by four waves, then the read of all, cost a second round
        // trip on those waves: 2,023 against 2,092 tokens/s without it.
        // shared-expert activations of every token: written in R, long landed by now
        // (T = 1 read them in G)
        if constexpr (TM != 1) {
            for (int i = tid; i < T * QE_FF_SH; i += NTH) {
                uint64_t w[1];
                read_tv<1>(EXr + EX_HSH + i, 0, tagR, w, true, pc);
                s_hsh[i] = tv_val(w[0]);
            }
        }
        __syncthreads();
        if (TM == 1 && wv == NWV - 1) {
            // weights and shared gate of the selection (read after the h wait), by a
            // wave the shared down rows leave idle
            // the selected experts' logit keys, written by the survivors in G (by tie key)
            const unsigned *s_full = (const unsigned *)(lds + L_TKF);
            auto tkey = [](int e) { return (e & 15) * 16 + (e >> 4); };
            const int myid = lane < QE_K_USED ? s_items[lane].x & (QE_N_EXPERT - 1) : s_items[0].x & (QE_N_EXPERT - 1);
            const float mine = ord2f(s_full[tkey(myid)]), sel0 = ord2f(s_full[tkey(s_items[0].x & (QE_N_EXPERT - 1))]);
            topk_finish(mine, myid, sel0, *(const float *)(lds + L_TK + 2048), lane, s_ids, s_wts, s_shg);
        }
        // The shared down rows of every D row group run first, while the routed
        // h is still on its way: wave (rr, half 0), 16-lane group g takes tokens
        // g, g + 4 of row rr.
        if (half == 0) {
            for (int m = 0; m < d_iters; ++m) {
                const int rb = (blockIdx.x + m * gridDim.x) * 8;
                if (rb >= QE_D) break;
                if (m > 0) {
                    const uint8_t *srow = sh_dn + (size_t)(rb + rr) * QE_SH_DN_ROW_BYTES;
                    dq0 = ((const uint4 *)(srow + l16 * 32))[0];
                    dq1 = ((const uint4 *)(srow + l16 * 32))[1];
                    dsc = ((const uint16_t *)(srow + QE_FF_SH))[l16];
                }
                float w8[32];
                unpack_i8x32(dq0, dq1, w8);
                const float ssd = f16_bits_to_f32(dsc);
                for (int t0 = 0; t0 < T; t0 += 4) {
                    const int t = t0 + isub;
                    float acc = 0.f;
                    if (t < T) {
#pragma unroll
                        for (int i = 0; i < 32; ++i) acc = fmaf(w8[i], s_hsh[t * QE_FF_SH + l16 * 32 + i], acc);
                    }
                    const float sd = sum16(acc * ssd);
                    if (l16 == 0 && t < T) s_sd[(m * 8 + rr) * DEC_T + t] = sd;
                }
            }
        }
        // T = 1: the first prefetched down block is decoded to int8 now, while h
        // is still on its way (about half the routed down's instructions)
        nl4_blk wpre;
        if constexpr (TM == 1) {
            wpre = nl4_decode_block<true>(dpq[0]);
#pragma unroll
            for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(wpre.w[i]));
        }
        if constexpr (TM == 1) {
            // Wave (item u = wv / 2, half hw = wv % 2) polls pair u's h words of its
            // half (elements 256 hw + 4 lane + 0..3), quantises them (8 lanes per
            // 32-block), and then its lane (row lane / 8, block 8 hw + lane % 8)
            // forms that block's dot with the item's down row: the routed down of a
            // wave waits for its own h only, with no workgroup barrier in between.
            const int u = wv >> 1, hw = wv & 1, b = 8 * hw + (lane & 7);
            static_assert(8 * QE_FF_EXP == 4 * NTH, "h of the 8 pairs: four words per thread");
            uint64_t w[4];
            read_tv_pairs<2>(EXr + EX_HF + 4 * tid, tagG, w, pc);
            float h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) h[i] = tv_val(w[i]);
            float am = fmaxf(fmaxf(fabsf(h[0]), fabsf(h[1])), fmaxf(fabsf(h[2]), fabsf(h[3])));
            am = fmaxf(am, dpp_f<QE_DPP_XOR1>(am));
            am = fmaxf(am, dpp_f<QE_DPP_XOR2>(am));
            am = fmaxf(am, dpp_f<QE_DPP_HMIRROR>(am));
            float dq;
            const float id = quant_scale_inv(am, dq);
            unsigned q = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) q |= (unsigned)(uint8_t)quant_one(h[i], id) << (8 * i);
            *(unsigned *)(s_hq + 4 * tid) = q;
            if ((tid & 7) == 0) s_hs[tid >> 3] = dq;
            // the other lanes' blocks of this half, written by this wave just above
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int8_t *hq = s_hq + u * QE_FF_EXP + b * 32;
            const uint4 h0 = *(const uint4 *)hq, h1 = *(const uint4 *)(hq + 16);
            const float hsc = s_hs[u * 16 + b];
            for (int m = 0; m < d_iters; ++m) {
                const int rb = (blockIdx.x + m * gridDim.x) * 8;
                if (rb >= QE_D) break;
                nl4_blk wq;
                uint16_t sraw;
                if (m == 0) { // prefetched during G, decoded before the h wait
                    wq = wpre;
                    sraw = (uint16_t)dps[0];
                } else {
                    const uint8_t *drow = arena + (size_t)(s_items[u].x & (QE_N_EXPERT - 1)) * QE_EXPERT_BYTES +
                                          QE_EXPERT_DOWN_OFF + (size_t)(rb + (lane >> 3)) * QE_DN_ROW_BYTES;
                    wq = nl4_decode_block<true>(*(const uint4 *)(drow + b * 16));
                    sraw = ((const uint16_t *)(drow + QE_FF_EXP / 2))[b];
                }
                const int P = nl4_block_dot(wq, h0, h1);
                float v = (f16_bits_to_f32(sraw) * hsc) * (float)P;
                v = v + dpp_f<QE_DPP_XOR1>(v); // the row's 8 blocks of this half
                v = v + dpp_f<QE_DPP_XOR2>(v);
                v = v + dpp_f<QE_DPP_HMIRROR>(v);
                if ((lane & 7) == 0) s_y[(u * 2 + hw) * 8 + (lane >> 3)] = v;
                __syncthreads();
                if (tid < 8) { // thread (row k): combine, items in k order
                    const int k = tid, ro = rb + k;
                    float yt = 0.f;
#pragma unroll
                    for (int it = 0; it < QE_K_USED; ++it) yt += s_wts[it] * (s_y[(it * 2) * 8 + k] + s_y[(it * 2 + 1) * 8 + k]);
                    const float sd = s_sd[(m * 8 + k) * DEC_T];
                    const float res = a.residual ? s_res[m * 8 + k] : 0.f;
                    const float out = (res + s_shg[0] * sd) + yt;
                    if (a.residual) s_res[m * 8 + k] = out; // the next layer's residual (its x)
                    if (last) {
                        a.x_out[ro] = out;
                        if (a.sd_out) a.sd_out[ro] = sd;
                    }
                    if (!last || EXN) { // the exit norm reads the last x like a next layer would
#pragma unroll
                        for (int r = 0; r < REP; ++r) ST_A(dst_x + r * EX_TOTAL + ro, pack_tv(out, tagD));
                        float *s_gx = (float *)(lds + L_GX);
                        s_gx[k] = out;
                        // the 8 rows' stores (lanes of wave 0) before lane 0 reads them
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        if (k == 0) {
                            const float g = sumsq_group8(s_gx);
#pragma unroll
                            for (int r = 0; r < REP; ++r) ST_A(dst_xs + r * EX_TOTAL + rb / 8, pack_tv(g, tagD));
                        }
                    }
                }
                __syncthreads(); // s_y is rewritten by the next row group
            }
        } else {
            for (int task = tid; task < np * 16; task += NTH) { // (pair, 32-block): 8 code words + 1 scale
                const int p = task >> 4, b = task & 15;
                uint64_t w[9];
                read_tv<9>(EXr + EX_HQ + ((size_t)p * 16 + b) * 9, 1, tagG, w, true, pc);
                uint4 *dq = (uint4 *)(s_hq + p * QE_FF_EXP + b * 32);
                dq[0] = make_uint4((unsigned)w[0], (unsigned)w[1], (unsigned)w[2], (unsigned)w[3]);
                dq[1] = make_uint4((unsigned)w[4], (unsigned)w[5], (unsigned)w[6], (unsigned)w[7]);
                s_hs[task] = tv_val(w[8]);
            }
            __syncthreads();
            for (int m = 0; m < d_iters; ++m) {
                const int rb = (blockIdx.x + m * gridDim.x) * 8;
                if (rb >= QE_D) break;
                const int r = rb + rr;
                // this lane group's per-token sums, in LDS: one add per pair (from the
                // group's first lane, in program order) instead of a select and an add
                // per token in every lane
                float *s_yg = (float *)(lds + L_YG) + (wv * 4 + isub) * DEC_T;
                if (l16 < DEC_T) s_yg[l16] = 0.f;
                // round k's down row block, loaded a round ahead (unconditionally: a
                // round past the items re-reads a valid row, never used, so the
                // compiler's waits stay per load); item round k = 0 came during G
                auto d_row = [&](int k, uint4 &q, unsigned &sr) {
                    const int u = half + 2 * (4 * k + isub);
                    const int4 it = s_items[u < nitems ? u : half];
                    const uint8_t *drow = arena + (size_t)it.x * QE_EXPERT_BYTES + QE_EXPERT_DOWN_OFF + (size_t)r * QE_DN_ROW_BYTES;
                    q = *(const uint4 *)(drow + l16 * 16);
                    sr = ((const uint16_t *)(drow + QE_FF_EXP / 2))[l16];
                };
                uint4 qn;
                unsigned sn;
                if (m == 0) { // prefetched during G
                    qn = dpq[0];
                    sn = dps[0];
                } else {
                    d_row(0, qn, sn);
                }
                for (int k = 0; half + 8 * k < nitems; ++k) {
                    const int s = 4 * k + isub, u = half + 2 * s;
                    const bool act = u < nitems;
                    const int4 it = s_items[act ? u : half];
                    const uint4 q = qn;
                    const uint16_t sraw = (uint16_t)sn;
                    d_row(k + 1, qn, sn);
                    nl4_blk w;
                    w = nl4_decode_block<false>(q); // at the register limit
                    const float sc = f16_bits_to_f32(sraw);
                    const int npair = act ? it.z : 0;
                    // pairs of the item (<= T), as many rounds as the wave's largest item
                    // needs (wave-uniform: the sums below are cross-lane)
                    for (int j = 0; j < T && __any(j < npair); ++j) {
                        const bool pj = j < npair;
                        const int p = pj ? s_pairs[it.y + j] : 0, tp = p / QE_K_USED;
                        const int8_t *hq = s_hq + p * QE_FF_EXP + l16 * 32;
                        const int P = nl4_block_dot(w, *(const uint4 *)hq, *(const uint4 *)(hq + 16));
                        const float v = sum16((sc * s_hs[p * 16 + l16]) * (float)P);
                        if (pj && l16 == 0)
                            __hip_atomic_fetch_add(s_yg + tp, v * s_wts[p], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                    }
                }
                if (lane < T) { // the wave's four lane groups, in order
                    const float *g = (const float *)(lds + L_YG) + wv * 4 * DEC_T + lane;
                    s_y[(rr * 2 + half) * DEC_T + lane] = ((g[0] + g[DEC_T]) + g[2 * DEC_T]) + g[3 * DEC_T];
                }
                __syncthreads();
                if (tid < 8 * T) { // thread (row, token): combine
                    const int k = tid / T, t = tid % T, ro = rb + k;
                    const float sd = s_sd[(m * 8 + k) * DEC_T + t];
                    const float yt = s_y[(k * 2) * DEC_T + t] + s_y[(k * 2 + 1) * DEC_T + t];
                    const float res = a.residual ? s_res[t * 32 + m * 8 + k] : 0.f;
                    const float out = (res + s_shg[t] * sd) + yt;
                    const size_t o = (size_t)t * QE_D + ro;
                    if (last) {
                        a.x_out[o] = out;
                        if (a.sd_out) a.sd_out[o] = sd;
                    }
                    if (!last || EXN) { // the exit norm reads the last x like a next layer would
#pragma unroll
                        for (int r = 0; r < REP; ++r) ST_A(dst_x + r * EX_TOTAL + o, pack_tv(out, tagD));
                        // the group's partial of the next norm's sum of squares (an fma
                        // chain over its 8 rows), gathered in LDS by the thread of row 0;
                        // these threads are all in wave 0, whose LDS accesses are ordered
                        float *s_gx = (float *)(lds + L_GX);
                        s_gx[t * 8 + k] = out;
                        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                        __builtin_amdgcn_wave_barrier();
                        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                        if (k == 0) {
                            const float g = sumsq_group8(s_gx + t * 8);
#pragma unroll
                            for (int r = 0; r < REP; ++r) ST_A(dst_xs + r * EX_TOTAL + t * 256 + rb / 8, pack_tv(g, tagD));
                        }
                    }
                }
                __syncthreads(); // s_y is rewritten by the next row group
            }
        }
        __syncthreads(); // the LDS union is rewritten by the next layer's R stage
    }

    // Routing sink of the last layer, written once at the end by workgroup 0, off
    // the layers' critical path, from what LDS still holds: the logits (kept in
    // G), ids / weights / shared gates (ids in rank order per token), pairs and
    // per-expert offsets in expert order (a stable counting sort: the slot of
    // pair p is the number of pairs with a smaller expert plus the earlier pairs
    // with the same one; T > 1 has it in s_pairs and the items, in expert order).
    if (blockIdx.x == 0) {
        const float *s_lgs = (const float *)(lds + L_LG);
        for (int i = threadIdx.x; i < T * QE_ROUTER_ROWS; i += NTH) a.logits[i] = s_lgs[i];
        if ((int)threadIdx.x < np) {
            const int p = threadIdx.x;
            a.ids[p] = s_ids[p];
            a.wts[p] = s_wts[p];
            if constexpr (TM == 1) {
                const int e = s_ids[p];
                int slot = 0;
#pragma unroll
                for (int q = 0; q < QE_K_USED; ++q) slot += s_ids[q] < e || (s_ids[q] == e && q < p);
                a.pairs[slot] = p;
            } else {
                a.pairs[p] = s_pairs[p]; // slot p
            }
        }
        if ((int)threadIdx.x < T) a.shg[threadIdx.x] = s_shg[threadIdx.x];
        if (threadIdx.x <= QE_N_EXPERT) {
            const int e = threadIdx.x;
            int o = 0;
            if constexpr (TM == 1) {
#pragma unroll
                for (int q = 0; q < QE_K_USED; ++q) o += s_ids[q] < e;
            } else { // first item (expert order) with an expert >= e: its first slot
                int lo = 0, hi = s_misc[0];
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (s_items[mid].x < e) lo = mid + 1; else hi = mid;
                }
                o = lo < s_misc[0] ? s_items[lo].y : np;
            }
            a.off[e] = o;
        }
    }

    // Exit norm (the next block's input norm, engine/qe.cpp:2243 / :2574):
    // workgroup t < T gathers token t of the last layer's x from the exchange
    // and writes RMSNorm(x) * exit_norm in the canonical order.
    if (EXN && (int)blockIdx.x < T) {
        const int t = blockIdx.x, li = a.n_layers - 1;
        const unsigned tagX = epoch * 65536u + (unsigned)li * 4u + 3u; // the last layer's tagD
        const uint64_t *src = EXr + EX_X + (size_t)(li & 1) * DEC_T * QE_D + (size_t)t * QE_D;
        for (int i = threadIdx.x; i < QE_D; i += NTH) {
            uint64_t w[1];
            read_tv<1>(src + i, 0, tagX, w, true, pc);
            s_xn[xpos(i)] = tv_val(w[0]);
        }
        __syncthreads();
        if (threadIdx.x < 64) {
            const int lane = threadIdx.x;
            float c[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) c[i] = s_xn[i * 65 + lane];
            const float ss = wave_sum_canon(sumsq_lane32(c));
            if (lane == 0) s_inv[0] = 1.0f / sqrtf(ss / (float)QE_D + QE_RMS_EPS);
        }
        __syncthreads();
        for (int e = threadIdx.x; e < QE_D; e += NTH)
            a.exit_xn[(size_t)t * QE_D + e] = (s_xn[xpos(e)] * s_inv[0]) * a.exit_norm[e];
    }

    // The last workgroup out advances the epoch, so the next launch uses new
    // tags.  Tags carry the epoch modulo 65536: a word that no launch rewrote
    // for exactly k * 65536 launches (EX_HF is written only by T = 1 launches,
    // EX_HQ only by T > 1, the slots of tokens >= T by larger batches) would
    // match a poll before its producer stores it.  So when the low 16 bits of
    // the epoch are about to wrap, the last workgroup out (every other one has
    // finished reading) zeroes the exchange: tag 0 is never expected (stage
    // numbers start at 1), and every word written after the wrap carries an
    // epoch that no earlier word of the same 65536-launch window holds.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) s_misc[2] = ADD_A(a.sync + SYNC_EXIT, 1u) == gridDim.x - 1;
    __syncthreads();
    if (s_misc[2]) {
        if (((epoch + 1u) & 0xffffu) == 0u) {
            for (size_t i = threadIdx.x; i < (size_t)QE_DECODE_EX_WORDS; i += NTH) ST_A(a.ex + i, (uint64_t)0);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        if (threadIdx.x == 0) {
            ST_A(a.sync + SYNC_EXIT, 0u);
            ST_A(a.sync + SYNC_EPOCH, epoch + 1u);
        }
    }
}

#define DEC_MAX_DEV 64
static std::mutex g_dec_setup_mu;

// The grid of each instantiation, per device (the current one): set up on its
// first launch there, with the kernel's dynamic LDS limit raised for that device.
template <int TM, bool EXN> static hipError_t launch_decode(const QeDecodeArgs &a, hipStream_t st) {
    static std::atomic<int> grids[DEC_MAX_DEV];
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= DEC_MAX_DEV) return hipErrorInvalidDevice;
    int grid = grids[dev].load(std::memory_order_acquire);
    if (!grid) {
        std::lock_guard<std::mutex> lk(g_dec_setup_mu);
        grid = grids[dev].load(std::memory_order_relaxed);
        if (!grid) {
            if ((e = hipFuncSetAttribute((const void *)k_decode<TM, EXN>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                         L_TOTAL)) != hipSuccess)
                return e;
            int cus = 0, per_cu = 0;
            if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
            if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode<TM, EXN>, NTH, L_TOTAL)) != hipSuccess)
                return e;
            if (per_cu < 1) return hipErrorInvalidConfiguration;
            // one workgroup per CU, 64..256 of them (a workgroup's D rows, <= 4 groups
            // of 8, stay within the 32-row residual buffer); per_cu is 1 (LDS), so the
            // grid is resident in full on an idle device
            grid = cus < 256 ? cus : 256;
            if (grid < DEC_MIN_GRID) return hipErrorInvalidConfiguration;
            grids[dev].store(grid, std::memory_order_release);
        }
    }
    void *args[] = {(void *)&a};
    return hipLaunchKernel((const void *)k_decode<TM, EXN>, dim3(grid), dim3(NTH), args, L_TOTAL, st);
}

hipError_t qe_launch_decode(const QeDecodeArgs &a, hipStream_t st) {
    if (a.T < 1 || a.T > DEC_T) return hipErrorInvalidValue;
    // the exit norm is a separate instantiation: its extra publication and tail
    // cost 1.5 % of the plain 40-layer stack when compiled in unused
    if (a.exit_xn) return a.T == 1 ? launch_decode<1, true>(a, st) : launch_decode<DEC_T, true>(a, st);
    return a.T == 1 ? launch_decode<1, false>(a, st) : launch_decode<DEC_T, false>(a, st);
}
