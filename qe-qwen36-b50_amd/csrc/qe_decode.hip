// Persistent decode kernel: T <= 8 tokens through n_layers MoE layers in ONE
// cooperative launch (the MoE sections of Engine::decode, engine/qe.cpp:2466-2572,
// and decode_multi<NT>, :1653-1737, looped over the layers as at :2241).
//
// Why persistent: on MI355X every kernel launch costs ~4.5 us of fixed
// duration (dispatch over 8 XCDs + end-of-kernel L2 write-back), while one
// B=1 layer moves 19.6 MB = 2.5 us at 8 TB/s.  Per layer this kernel runs
//   R  norm + router rows + shared gate|up row pairs   -> logits, silu(g)*u
//   G  top-8 + dispatch (every workgroup, redundantly), routed gate/up +
//      SwiGLU on 32-row units, quantised in place      -> int8 h + scales
//   D  routed down, shared down, combine, residual      -> next x
// Synchronisation is carried by the data: every value crossing workgroups is
// written as one 64-bit agent-scope store {value, tag}, where the tag names
// (launch epoch, layer, stage).  A consumer polls the entries it needs until
// every tag matches, so one store->load round trip both synchronises and
// delivers the data -- no barrier counters, no L2 write-back fences.  Agent
// scope makes the compiler emit sc1 loads/stores, coherent across the XCDs'
// separate L2s.  The dataflow orders buffer reuse: a producer can only start
// layer l+1's stage after every workgroup has consumed layer l's data of the
// same buffer (each stage needs contributions from every workgroup).
// Weights a stage will need and that do not depend on the data being waited
// for (router/shared rows, the down rows of the routed experts, the shared
// down row) are loaded into registers before the wait.
#include "qe_kernels.h"

#define LD_A(p) __hip_atomic_load((p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
#define ST_A(p, v) __hip_atomic_store((p), (v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
#define ADD_A(p, v) __hip_atomic_fetch_add((p), (v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)

#define DEC_T QE_SMALL_T
#define DEC_PFI 16        /* items whose down rows are prefetched into LDS during G */
#define SYNC_EPOCH 0
#define SYNC_EXIT 32
#define SYNC_CTR 64       /* 3 stages x 16 groups, 32 words apart: R, G, D */
#define SPIN_CAP (1 << 22)

#define DEC_MIN_GRID 64   /* D rows per workgroup stay <= 32 */

// LDS layout (bytes)
#define L_XQ 0                                      // int8 [T][2048]   quantised xn
#define L_XS (L_XQ + DEC_T * QE_D)                  // f32 [T][64]      its block scales
#define L_RES (L_XS + DEC_T * 64 * 4)               // f32 [T][32]      raw x of this workgroup's D rows
#define L_HSH (L_RES + DEC_T * 32 * 4)              // f32 [T][512]     shared-expert silu(g)*u
#define L_U (L_HSH + DEC_T * QE_FF_SH * 4)          // union, by stage:
#define L_XN L_U                                    //   R: f32 [T][32][64] xn, element-interleaved
#define L_H L_U                                     //   G: f32 [8][32] h of one 32-row unit
#define L_HQ L_U                                    //   D: int8 [T*8][512] quantised h
#define L_HS (L_HQ + DEC_T * 8 * QE_FF_EXP)         //   D: f32 [T*8][16] its block scales
#define L_U_END (L_U + DEC_T * QE_D * 4)
#define L_DW L_U_END                                // uint4 [4 waves][PFI][2 rows][16 blocks] down codes
#define L_DS (L_DW + 4 * DEC_PFI * 2 * 16 * 16)     // u32   [4 waves][PFI][2 rows][16 blocks] down scales
#define L_ITEMS (L_DS + 4 * DEC_PFI * 2 * 16 * 4)   // int4 [64]
#define L_PAIRS (L_ITEMS + 64 * 16)                 // int [64]
#define L_IDS (L_PAIRS + 64 * 4)                    // int [64]
#define L_WTS (L_IDS + 64 * 4)                      // f32 [64]
#define L_SHG (L_WTS + 64 * 4)                      // f32 [8]
#define L_MISC (L_SHG + 8 * 4)                      // int [16]
#define L_TOTAL (L_MISC + 16 * 4)
static_assert(L_HS + DEC_T * 8 * 16 * 4 <= L_U_END, "D-stage LDS must fit in the union");

// exchange buffer offsets (u64 words, {value or payload, tag})
#define EX_X 0                                      // 2 x [T][2048] f32
#define EX_L (EX_X + 2 * DEC_T * QE_D)              // [T][257] f32 logits
#define EX_HSH (EX_L + DEC_T * QE_ROUTER_ROWS)      // [T][512] f32 shared silu(g)*u
#define EX_HQ (EX_HSH + DEC_T * QE_FF_SH)           // [T*8][16][9]: 8 x int8x4, 1 x f32 scale
#define EX_TOTAL (EX_HQ + DEC_T * 8 * 16 * 9)
static_assert(EX_TOTAL == QE_DECODE_EX_WORDS, "exchange size must match the allocation");

QE_DEV uint64_t pack_tv(float v, unsigned tag) { return ((uint64_t)tag << 32) | __float_as_uint(v); }
QE_DEV float tv_val(uint64_t w) { return __uint_as_float((unsigned)w); }
QE_DEV bool tv_ok(uint64_t w, unsigned tag) { return (unsigned)(w >> 32) == tag; }

// Wave-uniform poll of N tagged entries per lane at src[i * stride]: reload
// until every lane sees `tag` on all of them (bounded; a timeout sets *err).
template <int N>
QE_DEV void poll_tv(const uint64_t *src, int stride, unsigned tag, float out[N], unsigned *err) {
    uint64_t w[N];
    for (int spins = 0;; ++spins) {
#pragma unroll
        for (int i = 0; i < N; ++i) w[i] = LD_A((uint64_t *)src + (size_t)i * stride);
        unsigned bad = 0;
#pragma unroll
        for (int i = 0; i < N; ++i) bad |= (unsigned)(w[i] >> 32) ^ tag;
        if (__all(bad == 0)) break;
        if (spins > SPIN_CAP) { ST_A(err, 1u); break; }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) out[i] = tv_val(w[i]);
}

// Stage counters: after issuing all of its tagged data stores a workgroup
// bumps its group's counter for the stage (groups of 16 workgroups; the add
// is posted, nothing waits on it).  A consumer's wave 0 polls the <= 16 group
// counters of the stage until each reaches 16 * (layer + 1), then every
// thread reads its data once (tags verified, rare retry).  Measured on
// MI355X with 256 workgroups: ~4.2 us per all-gather this way, against
// ~5.5 us polling one flag per workgroup and ~5.7 us polling the data itself.
QE_DEV void stage_arrive(unsigned *ctr) {
    __syncthreads();
    if (threadIdx.x == 0) (void)ADD_A(ctr + (blockIdx.x >> 4) * 32, 1u);
}
QE_DEV void stage_wait(const unsigned *ctr, unsigned round, unsigned *err) {
    if (threadIdx.x < 64) {
        const int g = threadIdx.x, ng = (gridDim.x + 15) >> 4;
        const unsigned gsz = (unsigned)((g + 1) * 16 <= (int)gridDim.x ? 16 : (int)gridDim.x - g * 16);
        for (int spins = 0;; ++spins) {
            const bool ok = g >= ng || LD_A((unsigned *)ctr + g * 32) >= gsz * round;
            if (__all(ok)) break;
            if (spins > SPIN_CAP) { ST_A(err, 1u); break; }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// Poll the 257 logits of one token in one round: v[j] = logit(lane + 64 j), v[4] = logit 256.
QE_DEV void poll_logits(const uint64_t *row, unsigned tag, float v[5], unsigned *err) {
    uint64_t w[5];
    for (int spins = 0;; ++spins) {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = LD_A((uint64_t *)row + threadIdx.x % 64 + 64 * j);
        w[4] = LD_A((uint64_t *)row + QE_N_EXPERT);
        unsigned bad = 0;
#pragma unroll
        for (int j = 0; j < 5; ++j) bad |= (unsigned)(w[j] >> 32) ^ tag;
        if (__all(bad == 0)) break;
        if (spins > SPIN_CAP) { ST_A(err, 1u); break; }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int j = 0; j < 5; ++j) v[j] = tv_val(w[j]);
}

// Order-preserving u32 image of a float (-0 folded onto +0 by the caller).
QE_DEV unsigned f2ord(float v) {
    const unsigned u = __float_as_uint(v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
QE_DEV float ord2f(unsigned o) { return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o); }

// top-8 of 256 logits held as v[j] = logit(lane + 64 j), the engine/qe.cpp:1454-1483
// order: larger value first, ties to the smaller (e % 16, e / 16).  Each candidate
// is one u64 {ordered value, 0xffff - key} so a wave max finds value and key together.
QE_DEV void wave_topk8(float v[4], float lg_sh, int lane, int *ids, float *wts, float *shg) {
    uint64_t c[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j, key = (e & 15) * 16 + (e >> 4);
        c[j] = ((uint64_t)f2ord(v[j] + 0.0f) << 32) | (unsigned)(0xffff - key);
    }
    float sel[QE_K_USED];
    int id[QE_K_USED];
#pragma unroll
    for (int k = 0; k < QE_K_USED; ++k) {
        uint64_t b = c[0];
#pragma unroll
        for (int j = 1; j < 4; ++j) b = c[j] > b ? c[j] : b;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint64_t o = ((uint64_t)(unsigned)__shfl_xor((int)(b >> 32), off, 64) << 32) |
                               (unsigned)__shfl_xor((int)(unsigned)b, off, 64);
            b = o > b ? o : b;
        }
        const int key = 0xffff - (int)(b & 0xffff);
        const int e = (key & 15) * 16 + (key >> 4);
        sel[k] = ord2f((unsigned)(b >> 32));
        id[k] = e;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (c[j] == b) c[j] = 0;
    }
    if (lane == 0) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < QE_K_USED; ++k) s += expf(sel[k] - sel[0]);
#pragma unroll
        for (int k = 0; k < QE_K_USED; ++k) {
            ids[k] = id[k];
            wts[k] = expf(sel[k] - sel[0]) / s;
        }
        *shg = 1.f / (1.f + expf(-lg_sh));
    }
}

__global__ __launch_bounds__(256) void k_decode(QeDecodeArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    int8_t *s_xq = (int8_t *)(lds + L_XQ);
    float *s_xs = (float *)(lds + L_XS);
    float *s_res = (float *)(lds + L_RES);
    float *s_hsh = (float *)(lds + L_HSH);
    float *s_xn = (float *)(lds + L_XN);
    float *s_h = (float *)(lds + L_H);
    int8_t *s_hq = (int8_t *)(lds + L_HQ);
    float *s_hs = (float *)(lds + L_HS);
    int4 *s_items = (int4 *)(lds + L_ITEMS);
    int *s_pairs = (int *)(lds + L_PAIRS);
    int *s_ids = (int *)(lds + L_IDS);
    float *s_wts = (float *)(lds + L_WTS);
    float *s_shg = (float *)(lds + L_SHG);
    int *s_misc = (int *)(lds + L_MISC);

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, l16 = lane & 15;
    const int T = a.T, np = T * QE_K_USED;
    const int nwaves = gridDim.x * 4, gw = blockIdx.x * 4 + wv;
    const int n_rtask = QE_ROUTER_ROWS + QE_FF_SH; // router rows, then shared (gate, up) row pairs
    const int d_iters = (QE_D / 8 + gridDim.x - 1) / gridDim.x; // D row groups of 8 per workgroup
    if (tid == 0) s_misc[1] = (int)LD_A(a.sync + SYNC_EPOCH);
    __syncthreads();
    const unsigned epoch = (unsigned)s_misc[1];
    uint64_t *EX = a.ex;
    unsigned *CR = a.sync + SYNC_CTR, *CG = CR + 16 * 32, *CD = CG + 16 * 32;

    for (int li = 0; li < a.n_layers; ++li) {
        const int l = a.first_layer + li;
        const bool last = li == a.n_layers - 1;
        const unsigned tagR = epoch * 65536u + (unsigned)li * 4u + 1u; // logits, shared h
        const unsigned tagG = tagR + 1u;                               // routed int8 h
        const unsigned tagD = tagR + 2u;                               // x of the next layer
        const unsigned tagIn = tagR - 2u;                              // x of this layer (li > 0)
        const uint64_t *src_x = EX + EX_X + (size_t)((li - 1) & 1) * DEC_T * QE_D;
        uint64_t *dst_x = EX + EX_X + (size_t)(li & 1) * DEC_T * QE_D;
        const uint8_t *arena = a.arena + (size_t)l * QE_LAYER_EXPERT_BYTES;
        const float *router = a.router + (size_t)l * QE_ROUTER_ROWS * QE_D;
        const float *bias = a.bias_on[l] ? a.bias + (size_t)l * QE_N_EXPERT : nullptr;
        const uint8_t *sh_gu = a.sh_gu + (size_t)l * QE_SH_GU_BYTES;
        const uint8_t *sh_dn = a.sh_dn + (size_t)l * QE_SH_DN_BYTES;
        const float *pnorm = a.norm ? a.post_norm + (size_t)l * QE_D : nullptr;

        // ================= R: router rows + shared (gate, up) pairs =================
        // first task's weights into registers before waiting for x
        const int task0 = gw;
        float wr[32];
        uint4 g0 = make_uint4(0, 0, 0, 0), g1 = g0, u0 = g0, u1 = g0;
        float gsc = 0.f, usc = 0.f;
        auto load_task = [&](int task) {
            if (task < QE_ROUTER_ROWS) {
                load32(router + (size_t)task * QE_D + lane * 32, wr);
            } else if (task < n_rtask) {
                const int j = task - QE_ROUTER_ROWS;
                const uint8_t *rg = sh_gu + (size_t)j * QE_SH_GU_ROW_BYTES, *ru = sh_gu + (size_t)(QE_FF_SH + j) * QE_SH_GU_ROW_BYTES;
                g0 = ((const uint4 *)(rg + lane * 32))[0];
                g1 = ((const uint4 *)(rg + lane * 32))[1];
                gsc = f16_bits_to_f32(((const uint16_t *)(rg + QE_D))[lane]);
                u0 = ((const uint4 *)(ru + lane * 32))[0];
                u1 = ((const uint4 *)(ru + lane * 32))[1];
                usc = f16_bits_to_f32(((const uint16_t *)(ru + QE_D))[lane]);
            }
        };
        load_task(task0);
        if (li > 0) stage_wait(CD, (unsigned)li, a.err);
        for (int t = wv; t < T; t += 4) {
            float v[32];
            if (li == 0) load32(a.x_in + (size_t)t * QE_D + lane * 32, v);
            else poll_tv<32>(src_x + (size_t)t * QE_D + lane * 32, 1, tagIn, v, a.err);
            if (a.residual) { // raw x of this workgroup's D rows, 8 per group, all inside one 32-chunk
                for (int m = 0; m < d_iters; ++m) {
                    const int rb = (blockIdx.x + m * gridDim.x) * 8;
                    if (rb < QE_D && (rb >> 5) == lane) {
                        const int o = rb & 31;
#pragma unroll
                        for (int i = 0; i < 8; ++i)
                            s_res[t * 32 + m * 8 + i] = o == 0 ? v[i] : o == 8 ? v[8 + i] : o == 16 ? v[16 + i] : v[24 + i];
                    }
                }
            }
            wave_norm_chunk(v, pnorm, lane);
#pragma unroll
            for (int i = 0; i < 32; ++i) s_xn[t * QE_D + i * 64 + lane] = v[i];
            lane_quant_store(v, s_xq + t * QE_D + lane * 32, s_xs + t * 64 + lane);
            if (last && blockIdx.x == 0 && a.xn_out) {
#pragma unroll
                for (int i = 0; i < 32; ++i) a.xn_out[(size_t)t * QE_D + lane * 32 + i] = v[i];
            }
        }
        __syncthreads();
        for (int task = task0; task < n_rtask; task += nwaves) {
            if (task != task0) load_task(task);
            if (task < QE_ROUTER_ROWS) {
                const bool add_bias = bias && task < QE_N_EXPERT;
                const float b = add_bias ? bias[task] : 0.f;
                for (int t = 0; t < T; ++t) {
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) acc = fmaf(wr[i], s_xn[t * QE_D + i * 64 + lane], acc);
                    acc = wave_sum_canon(acc);
                    if (lane == 0) ST_A(EX + EX_L + t * QE_ROUTER_ROWS + task, pack_tv(add_bias ? acc + b : acc, tagR));
                }
            } else {
                const int j = task - QE_ROUTER_ROWS;
                float wg[32], wu[32];
                unpack_i8x32(g0, g1, wg);
                unpack_i8x32(u0, u1, wu);
                for (int t = 0; t < T; ++t) {
                    float ag = 0.f, au = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) {
                        const float xv = s_xn[t * QE_D + i * 64 + lane];
                        ag = fmaf(wg[i], xv, ag);
                        au = fmaf(wu[i], xv, au);
                    }
                    ag = wave_sum_canon(ag * gsc);
                    au = wave_sum_canon(au * usc);
                    if (lane == 0) ST_A(EX + EX_HSH + t * QE_FF_SH + j, pack_tv(silu_mul(ag, au), tagR));
                }
            }
        }
        stage_arrive(CR);

        // ================= G: top-8, dispatch, routed gate/up =================
        stage_wait(CR, (unsigned)li + 1u, a.err);
        for (int t = wv; t < T; t += 4) {
            float v[5];
            poll_logits(EX + EX_L + t * QE_ROUTER_ROWS, tagR, v, a.err);
            if (last && blockIdx.x == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) a.logits[t * QE_ROUTER_ROWS + lane + 64 * j] = v[j];
                if (lane == 0) a.logits[t * QE_ROUTER_ROWS + QE_N_EXPERT] = v[4];
            }
            wave_topk8(v, v[4], lane, s_ids + t * QE_K_USED, s_wts + t * QE_K_USED, s_shg + t);
        }
        for (int t = 0; t < T; ++t) { // shared-expert activations of token t, used in D
            float hv[2];
            poll_tv<2>(EX + EX_HSH + t * QE_FF_SH + tid, 256, tagR, hv, a.err);
            s_hsh[t * QE_FF_SH + tid] = hv[0];
            s_hsh[t * QE_FF_SH + 256 + tid] = hv[1];
        }
        __syncthreads();
        if (wv == 0) {
            // stable counting sort of the T*8 pairs by expert (engine/qe.cpp:1965-1976):
            // slot of pair p = #pairs with a smaller expert + #earlier pairs with the same one
            const int e = lane < np ? s_ids[lane] : 1 << 20;
            int lt = 0, rank = 0, cnt = 0;
            for (int q = 0; q < np; ++q) {
                const int f = s_ids[q];
                lt += f < e;
                cnt += f == e;
                rank += (f == e) & (q < lane);
            }
            const bool first = lane < np && rank == 0;
            const unsigned long long fm = __ballot(first);
            int item = 0;
            for (int q = 0; q < np; ++q) item += (int)((fm >> q) & 1ull) & (s_ids[q] < e);
            if (lane < np) s_pairs[lt + rank] = lane;
            if (first) s_items[item] = make_int4(e, lt, cnt, 0);
            if (lane == 0) s_misc[0] = __popcll(fm);
            if (last && blockIdx.x == 0) {
                if (lane < np) {
                    a.pairs[lt + rank] = lane;
                    a.ids[lane] = e;
                    a.wts[lane] = s_wts[lane];
                }
                if (lane < T) a.shg[lane] = s_shg[lane];
#pragma unroll
                for (int k = 0; k < 4; ++k) { // per-expert offsets for the routing sink
                    const int ee = lane * 4 + k;
                    int o = 0;
                    for (int q = 0; q < np; ++q) o += s_ids[q] < ee;
                    a.off[ee] = o;
                }
                if (lane == 0) a.off[QE_N_EXPERT] = np;
            }
        }
        __syncthreads();
        const int nitems = s_misc[0];

        // down rows of this workgroup's first D group (2 per wave) for the first DEC_PFI items:
        // asynchronous global->LDS copies issued now, consumed after the G stage
        const int rd0 = blockIdx.x * 8 + wv * 2;
        const int pf_items = nitems < DEC_PFI ? nitems : DEC_PFI;
        uint4 *s_dw = (uint4 *)(lds + L_DW) + wv * DEC_PFI * 32;
        // a sub-dword global->LDS load stores each lane's value zero-extended into its own dword
        unsigned *s_ds = (unsigned *)(lds + L_DS) + wv * DEC_PFI * 32;
        for (int u0 = 0; u0 < pf_items; u0 += 2) {
            const int sub = lane >> 5, u = u0 + sub < pf_items ? u0 + sub : u0; // lane -> (item, row, block)
            const uint8_t *drow = arena + (size_t)s_items[u].x * QE_EXPERT_BYTES + QE_EXPERT_DOWN_OFF +
                                  (size_t)(rd0 + ((lane >> 4) & 1)) * QE_DN_ROW_BYTES;
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(drow + l16 * 16),
                                             (__attribute__((address_space(3))) void *)(s_dw + u0 * 32), 16, 0, 0);
            __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)(drow + QE_FF_EXP / 2 + l16 * 2),
                                             (__attribute__((address_space(3))) void *)(s_ds + u0 * 32), 2, 0, 0);
        }
        const int half = (lane >> 4) & 1, rsel = lane >> 5;
        uint4 dq0 = make_uint4(0, 0, 0, 0), dq1 = dq0; // shared down row of the first D group
        uint16_t dsc = 0;
        {
            const uint8_t *srow = sh_dn + (size_t)(rd0 + rsel) * QE_SH_DN_ROW_BYTES;
            dq0 = ((const uint4 *)(srow + l16 * 32))[0];
            dq1 = ((const uint4 *)(srow + l16 * 32))[1];
            dsc = ((const uint16_t *)(srow + QE_FF_SH))[l16];
        }

        // units: (item, 32-row block); wave w takes 8 rows, 8 lanes per row, lane owns blocks lb + 8 j
        const int lb = lane & 7, rl = wv * 8 + (lane >> 3);
        for (int unit = blockIdx.x; unit < nitems * 16; unit += gridDim.x) {
            const int4 it = s_items[unit >> 4];
            const int blk32 = unit & 15, r = blk32 * 32 + rl;
            const uint8_t *base = arena + (size_t)it.x * QE_EXPERT_BYTES;
            const uint8_t *rg = base + (size_t)r * QE_GU_ROW_BYTES, *ru = base + (size_t)(QE_FF_EXP + r) * QE_GU_ROW_BYTES;
            nl4_blk dg[8], du[8];
            float sg[8], su[8];
            {
                uint4 qg[8], qu[8];
                uint16_t sgr[8], sur[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int b = lb + 8 * j;
                    qg[j] = *(const uint4 *)(rg + b * 16);
                    qu[j] = *(const uint4 *)(ru + b * 16);
                    sgr[j] = ((const uint16_t *)(rg + QE_D / 2))[b];
                    sur[j] = ((const uint16_t *)(ru + QE_D / 2))[b];
                }
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    dg[j] = nl4_decode_block(qg[j]);
                    du[j] = nl4_decode_block(qu[j]);
                    sg[j] = f16_bits_to_f32(sgr[j]);
                    su[j] = f16_bits_to_f32(sur[j]);
                }
            }
            for (int jp = 0; jp < it.z; ++jp) {
                const int t = s_pairs[it.y + jp] / QE_K_USED;
                float G = 0.f, U = 0.f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int b = lb + 8 * j;
                    const uint4 x0 = *(const uint4 *)(s_xq + t * QE_D + b * 32), x1 = *(const uint4 *)(s_xq + t * QE_D + b * 32 + 16);
                    const float xsv = s_xs[t * 64 + b];
                    G = fmaf(sg[j] * xsv, (float)nl4_block_dot(dg[j], x0, x1), G);
                    U = fmaf(su[j] * xsv, (float)nl4_block_dot(du[j], x0, x1), U);
                }
#pragma unroll
                for (int off = 1; off < 8; off <<= 1) {
                    G = G + __shfl_xor(G, off, 64);
                    U = U + __shfl_xor(U, off, 64);
                }
                if (lb == 0) s_h[jp * 32 + rl] = silu_mul(G, U);
            }
            __syncthreads();
            { // quantise the unit's 32-row block of every pair: thread (pair jp, row rr)
                const int jp = tid >> 5, rr = tid & 31;
                const bool act = jp < it.z;
                const float hv = act ? s_h[jp * 32 + rr] : 0.f;
                float amax = fabsf(hv);
#pragma unroll
                for (int off = 1; off < 32; off <<= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
                float d;
                const float id = quant_scale_inv(amax, d);
                const unsigned q = (unsigned)(uint8_t)quant_one(hv, id);
                const unsigned q1 = __shfl_down(q, 1, 64), q2 = __shfl_down(q, 2, 64), q3 = __shfl_down(q, 3, 64);
                if (act) {
                    const int p = s_pairs[it.y + jp];
                    uint64_t *dstw = EX + EX_HQ + ((size_t)p * 16 + blk32) * 9;
                    if ((rr & 3) == 0) ST_A(dstw + (rr >> 2), ((uint64_t)tagG << 32) | (q | (q1 << 8) | (q2 << 16) | (q3 << 24)));
                    if (rr == 0) ST_A(dstw + 8, pack_tv(d, tagG));
                }
            }
            __syncthreads(); // s_h is reused by the next unit
        }
        stage_arrive(CG);

        // ================= D: routed down + shared down + combine =================
        stage_wait(CG, (unsigned)li + 1u, a.err);
        for (int task = tid; task < np * 16; task += 256) { // (pair, 32-block): 8 code words + 1 scale
            const int p = task >> 4, b = task & 15;
            const uint64_t *srcw = EX + EX_HQ + ((size_t)p * 16 + b) * 9;
            uint64_t w[9];
            for (int spins = 0;; ++spins) {
#pragma unroll
                for (int i = 0; i < 9; ++i) w[i] = LD_A((uint64_t *)srcw + i);
                unsigned bad = 0;
#pragma unroll
                for (int i = 0; i < 9; ++i) bad |= (unsigned)(w[i] >> 32) ^ tagG;
                if (__all(bad == 0)) break;
                if (spins > SPIN_CAP) { ST_A(a.err, 1u); break; }
                __builtin_amdgcn_s_sleep(1);
            }
            uint4 *dq = (uint4 *)(s_hq + p * QE_FF_EXP + b * 32);
            dq[0] = make_uint4((unsigned)w[0], (unsigned)w[1], (unsigned)w[2], (unsigned)w[3]);
            dq[1] = make_uint4((unsigned)w[4], (unsigned)w[5], (unsigned)w[6], (unsigned)w[7]);
            s_hs[task] = tv_val(w[8]);
        }
        __builtin_amdgcn_s_waitcnt(0); // this wave's global->LDS prefetch has landed
        __syncthreads();
        for (int m = 0; m < d_iters; ++m) {
            const int rb = (blockIdx.x + m * gridDim.x) * 8;
            if (rb >= QE_D) break;
            const int r = rb + wv * 2 + rsel;
            float y[DEC_T];
#pragma unroll
            for (int t = 0; t < DEC_T; ++t) y[t] = 0.f;
            for (int u = half; u < nitems; u += 2) {
                const int4 it = s_items[u];
                uint4 q;
                uint16_t sraw;
                if (m == 0 && u < DEC_PFI) {
                    q = s_dw[u * 32 + rsel * 16 + l16];
                    sraw = (uint16_t)s_ds[u * 32 + rsel * 16 + l16];
                } else {
                    const uint8_t *drow = arena + (size_t)it.x * QE_EXPERT_BYTES + QE_EXPERT_DOWN_OFF + (size_t)r * QE_DN_ROW_BYTES;
                    q = *(const uint4 *)(drow + l16 * 16);
                    sraw = ((const uint16_t *)(drow + QE_FF_EXP / 2))[l16];
                }
                const nl4_blk w = nl4_decode_block(q);
                const float sc = f16_bits_to_f32(sraw);
                for (int j = 0; j < it.z; ++j) {
                    const int p = s_pairs[it.y + j], tp = p / QE_K_USED;
                    const int8_t *hq = s_hq + p * QE_FF_EXP + l16 * 32;
                    const int P = nl4_block_dot(w, *(const uint4 *)hq, *(const uint4 *)(hq + 16));
                    float v = (sc * s_hs[p * 16 + l16]) * (float)P;
                    v = sum16(v) * s_wts[p];
#pragma unroll
                    for (int t = 0; t < DEC_T; ++t) y[t] += t == tp ? v : 0.f;
                }
            }
#pragma unroll
            for (int t = 0; t < DEC_T; ++t) y[t] = y[t] + __shfl_xor(y[t], 16, 64);
            if (m > 0) {
                const uint8_t *srow = sh_dn + (size_t)r * QE_SH_DN_ROW_BYTES;
                dq0 = ((const uint4 *)(srow + l16 * 32))[0];
                dq1 = ((const uint4 *)(srow + l16 * 32))[1];
                dsc = ((const uint16_t *)(srow + QE_FF_SH))[l16];
            }
            float w8[32];
            unpack_i8x32(dq0, dq1, w8);
            const float ssd = f16_bits_to_f32(dsc);
            for (int t = 0; t < T; ++t) {
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) acc = fmaf(w8[i], s_hsh[t * QE_FF_SH + l16 * 32 + i], acc);
                const float sd = sum16(acc * ssd);
                float yt = y[0];
#pragma unroll
                for (int k = 1; k < DEC_T; ++k) yt = t == k ? y[k] : yt;
                if ((lane & 31) == 0) {
                    const size_t o = (size_t)t * QE_D + r;
                    const float res = a.residual ? s_res[t * 32 + m * 8 + (r - rb)] : 0.f;
                    const float out = (res + s_shg[t] * sd) + yt;
                    if (last) {
                        a.x_out[o] = out;
                        if (a.sd_out) a.sd_out[o] = sd;
                    } else {
                        ST_A(dst_x + o, pack_tv(out, tagD));
                    }
                }
            }
        }
        if (!last) stage_arrive(CD);
        __syncthreads(); // the LDS union is rewritten by the next layer's R stage
    }

    // the last workgroup out clears the stage counters and advances the epoch,
    // so the next launch starts from zero counts with new tags
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0 && ADD_A(a.sync + SYNC_EXIT, 1u) == gridDim.x - 1) {
        for (int i = 0; i < 3 * 16; ++i) ST_A(a.sync + SYNC_CTR + i * 32, 0u);
        ST_A(a.sync + SYNC_EXIT, 0u);
        ST_A(a.sync + SYNC_EPOCH, epoch + 1u);
    }
}

hipError_t qe_launch_decode(const QeDecodeArgs &a, hipStream_t st) {
    static int grid = 0;
    if (!grid) {
        hipError_t e = hipFuncSetAttribute((const void *)k_decode, hipFuncAttributeMaxDynamicSharedMemorySize, L_TOTAL);
        if (e != hipSuccess) return e;
        int dev = 0, cus = 0, per_cu = 0;
        if ((e = hipGetDevice(&dev)) != hipSuccess) return e;
        if ((e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess) return e;
        if ((e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_decode, 256, L_TOTAL)) != hipSuccess) return e;
        if (per_cu < 1) return hipErrorInvalidConfiguration;
        // one workgroup per CU, 64..256 of them (stage counters cover 16 groups of 16; D
        // rows per workgroup stay within the 32-row residual buffer)
        grid = cus < 256 ? cus : 256;
        if (grid < DEC_MIN_GRID) return hipErrorInvalidConfiguration;
    }
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)k_decode, dim3(grid), dim3(256), args, L_TOTAL, st);
}
