// Persistent decode kernel: T <= 8 tokens through n_layers MoE layers in ONE
// cooperative launch (the MoE sections of Engine::decode, engine/qe.cpp:2466-2572,
// and decode_multi<NT>, :1653-1737, looped over the layers as at :2241).
//
// Why persistent: on MI355X every kernel launch costs ~4.5 us of fixed
// duration (dispatch over 8 XCDs + end-of-kernel L2 write-back), while one
// B=1 layer moves 19.6 MB = 2.5 us at 8 TB/s.  Per layer this kernel runs
//   R  norm + router rows + shared gate|up rows            -> logits, shgu
//   G  top-8 + dispatch (every workgroup, redundantly), routed gate/up + SwiGLU -> h
//   D  quantise h, routed down, shared down, combine, residual -> next x
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
#define DEC_PF 8          /* routed down rows prefetched per lane (items u = half, half+2, ...) */
#define SYNC_EPOCH 0
#define SYNC_EXIT 32
#define SYNC_FLAGS 64     /* 3 x 256 per-workgroup stage flags: R, G, D */
#define SPIN_CAP (1 << 22)

// LDS layout (bytes)
#define L_XQ 0                                      // int8 [T][2048]
#define L_XS (L_XQ + DEC_T * QE_D)                  // f32 [T][64]
#define L_U (L_XS + DEC_T * 64 * 4)                 // union: R xn f32 [T][32][64] | D hq/hs/hsh
#define L_HQ L_U                                    // int8 [T*8][512]
#define L_HS (L_HQ + DEC_T * 8 * QE_FF_EXP)         // f32 [T*8][16]
#define L_HSH (L_HS + DEC_T * 8 * 16 * 4)           // f32 [T][512]
#define L_U_END (L_U + DEC_T * QE_D * 4)
#define L_ITEMS L_U_END                             // int4 [64]
#define L_PAIRS (L_ITEMS + 64 * 16)                 // int [64]
#define L_IDS (L_PAIRS + 64 * 4)                    // int [64]
#define L_WTS (L_IDS + 64 * 4)                      // f32 [64]
#define L_SHG (L_WTS + 64 * 4)                      // f32 [8]
#define L_FIRST (L_SHG + 8 * 4)                     // int [64]
#define L_MISC (L_FIRST + 64 * 4)                   // int [16]
#define L_TOTAL (L_MISC + 16 * 4)
static_assert(L_HSH + DEC_T * QE_FF_SH * 4 <= L_U_END, "D-stage LDS must fit in the union");

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

// Stage flags: a producer workgroup stores its flag (the stage tag) after
// issuing all of its tagged data stores; a consumer's wave 0 polls the 1 KB of
// flags, then every thread reads its data once (tags verified, rare retry).
// Polling the flags instead of the data keeps spinning workgroups from
// flooding the memory system that the producers are still streaming from.
QE_DEV void set_flag(unsigned *flags, unsigned tag) {
    __syncthreads();
    if (threadIdx.x == 0) ST_A(flags + blockIdx.x, tag);
}
QE_DEV void wait_flags(const unsigned *flags, unsigned tag, unsigned *err) {
    if (threadIdx.x < 64) {
        for (int spins = 0;; ++spins) {
            bool ok = true;
            for (int i = threadIdx.x; i < (int)gridDim.x; i += 64) ok = ok && LD_A((unsigned *)flags + i) == tag;
            if (__all(ok)) break;
            if (spins > SPIN_CAP) { ST_A(err, 1u); break; }
            __builtin_amdgcn_s_sleep(2);
        }
    }
    __syncthreads();
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
    float *s_xn = (float *)(lds + L_U);
    int8_t *s_hq = (int8_t *)(lds + L_HQ);
    float *s_hs = (float *)(lds + L_HS);
    float *s_hsh = (float *)(lds + L_HSH);
    int4 *s_items = (int4 *)(lds + L_ITEMS);
    int *s_pairs = (int *)(lds + L_PAIRS);
    int *s_ids = (int *)(lds + L_IDS);
    float *s_wts = (float *)(lds + L_WTS);
    float *s_shg = (float *)(lds + L_SHG);
    int *s_first = (int *)(lds + L_FIRST);
    int *s_misc = (int *)(lds + L_MISC);

    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, l16 = lane & 15;
    const int T = a.T, np = T * QE_K_USED;
    const int nwaves = gridDim.x * 4, gw = blockIdx.x * 4 + wv;
    if (tid == 0) s_misc[1] = (int)LD_A(a.sync + SYNC_EPOCH);
    __syncthreads();
    const unsigned epoch = (unsigned)s_misc[1];
    const uint64_t *EXX = a.ex_x, *EXL = a.ex_logits, *EXS = a.ex_shgu, *EXH = a.ex_h;
    unsigned *FR = a.sync + SYNC_FLAGS, *FG = FR + 256, *FD = FG + 256;

    for (int li = 0; li < a.n_layers; ++li) {
        const int l = a.first_layer + li;
        const bool last = li == a.n_layers - 1;
        const unsigned tagR = epoch * 65536u + (unsigned)li * 4u + 1u; // logits, shgu
        const unsigned tagG = tagR + 1u;                               // h
        const unsigned tagD = tagR + 2u;                               // x of the next layer
        const unsigned tagIn = tagR - 2u;                              // x of this layer (li > 0)
        const uint64_t *src_x = EXX + (size_t)((li - 1) & 1) * DEC_T * QE_D;
        uint64_t *dst_x = (uint64_t *)EXX + (size_t)(li & 1) * DEC_T * QE_D;
        const uint8_t *arena = a.arena + (size_t)l * QE_LAYER_EXPERT_BYTES;
        const float *router = a.router + (size_t)l * QE_ROUTER_ROWS * QE_D;
        const float *bias = a.bias_on[l] ? a.bias + (size_t)l * QE_N_EXPERT : nullptr;
        const uint8_t *sh_gu = a.sh_gu + (size_t)l * QE_SH_GU_BYTES;
        const uint8_t *sh_dn = a.sh_dn + (size_t)l * QE_SH_DN_BYTES;
        const float *pnorm = a.norm ? a.post_norm + (size_t)l * QE_D : nullptr;

        // ================= R: router + shared gate|up =================
        // this wave's rows (gw, gw + nwaves): weights into registers before waiting for x
        const int row0 = gw, row1 = gw + nwaves;
        float wr[32];
        uint4 sq0 = make_uint4(0, 0, 0, 0), sq1 = sq0, tq0 = sq0, tq1 = sq0;
        float ssc = 0.f, tsc = 0.f;
        if (row0 < QE_ROUTER_ROWS) {
            load32(router + (size_t)row0 * QE_D + lane * 32, wr);
        } else if (row0 < QE_ROUTER_ROWS + QE_SH_GU_ROWS) {
            const uint8_t *rp = sh_gu + (size_t)(row0 - QE_ROUTER_ROWS) * QE_SH_GU_ROW_BYTES;
            sq0 = ((const uint4 *)(rp + lane * 32))[0];
            sq1 = ((const uint4 *)(rp + lane * 32))[1];
            ssc = f16_bits_to_f32(((const uint16_t *)(rp + QE_D))[lane]);
        }
        if (row1 >= QE_ROUTER_ROWS && row1 < QE_ROUTER_ROWS + QE_SH_GU_ROWS) {
            const uint8_t *rp = sh_gu + (size_t)(row1 - QE_ROUTER_ROWS) * QE_SH_GU_ROW_BYTES;
            tq0 = ((const uint4 *)(rp + lane * 32))[0];
            tq1 = ((const uint4 *)(rp + lane * 32))[1];
            tsc = f16_bits_to_f32(((const uint16_t *)(rp + QE_D))[lane]);
        }
        if (li > 0) wait_flags(FD, tagIn, a.err);
        for (int t = wv; t < T; t += 4) {
            float v[32];
            if (li == 0) load32(a.x_in + (size_t)t * QE_D + lane * 32, v);
            else poll_tv<32>(src_x + (size_t)t * QE_D + lane * 32, 1, tagIn, v, a.err);
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
        for (int row = row0; row < QE_ROUTER_ROWS + QE_SH_GU_ROWS; row += nwaves) {
            if (row > row1) { // rows beyond the two prefetched ones (small grids only)
                if (row < QE_ROUTER_ROWS) {
                    load32(router + (size_t)row * QE_D + lane * 32, wr);
                } else {
                    const uint8_t *rp = sh_gu + (size_t)(row - QE_ROUTER_ROWS) * QE_SH_GU_ROW_BYTES;
                    tq0 = ((const uint4 *)(rp + lane * 32))[0];
                    tq1 = ((const uint4 *)(rp + lane * 32))[1];
                    tsc = f16_bits_to_f32(((const uint16_t *)(rp + QE_D))[lane]);
                }
            }
            if (row < QE_ROUTER_ROWS) {
                if (row == row1) load32(router + (size_t)row * QE_D + lane * 32, wr);
                const bool add_bias = bias && row < QE_N_EXPERT;
                const float b = add_bias ? bias[row] : 0.f;
                for (int t = 0; t < T; ++t) {
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) acc = fmaf(wr[i], s_xn[t * QE_D + i * 64 + lane], acc);
                    acc = wave_sum_canon(acc);
                    if (lane == 0)
                        ST_A((uint64_t *)EXL + t * QE_ROUTER_ROWS + row, pack_tv(add_bias ? acc + b : acc, tagR));
                }
            } else {
                float w[32];
                const bool first = row == row0;
                unpack_i8x32(first ? sq0 : tq0, first ? sq1 : tq1, w);
                const float sc = first ? ssc : tsc;
                const int r = row - QE_ROUTER_ROWS;
                for (int t = 0; t < T; ++t) {
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < 32; ++i) acc = fmaf(w[i], s_xn[t * QE_D + i * 64 + lane], acc);
                    acc = wave_sum_canon(acc * sc);
                    if (lane == 0) ST_A((uint64_t *)EXS + t * QE_SH_GU_ROWS + r, pack_tv(acc, tagR));
                }
            }
        }

        set_flag(FR, tagR);
        // ================= G: top-8, dispatch, routed gate/up =================
        wait_flags(FR, tagR, a.err);
        for (int t = wv; t < T; t += 4) {
            float v[4], lsh[1];
            poll_tv<4>(EXL + t * QE_ROUTER_ROWS + lane, 64, tagR, v, a.err);
            poll_tv<1>(EXL + t * QE_ROUTER_ROWS + QE_N_EXPERT, 0, tagR, lsh, a.err);
            if (last && blockIdx.x == 0) {
#pragma unroll
                for (int j = 0; j < 4; ++j) a.logits[t * QE_ROUTER_ROWS + lane + 64 * j] = v[j];
                if (lane == 0) a.logits[t * QE_ROUTER_ROWS + QE_N_EXPERT] = lsh[0];
            }
            wave_topk8(v, lsh[0], lane, s_ids + t * QE_K_USED, s_wts + t * QE_K_USED, s_shg + t);
        }
        __syncthreads();
        // stable counting sort of the T*8 pairs by expert (engine/qe.cpp:1965-1976):
        // position = #pairs with a smaller expert + #earlier pairs with the same one
        if (tid < np) {
            const int e = s_ids[tid];
            int lt = 0, rank = 0;
            for (int q = 0; q < np; ++q) {
                const int f = s_ids[q];
                lt += f < e;
                rank += (f == e) & (q < tid);
            }
            s_pairs[lt + rank] = tid;
            s_first[tid] = rank == 0;
            if (last && blockIdx.x == 0) {
                a.pairs[lt + rank] = tid;
                a.ids[tid] = e;
                a.wts[tid] = s_wts[tid];
                if (tid < T) a.shg[tid] = s_shg[tid];
            }
        }
        __syncthreads();
        if (tid < np && s_first[tid]) {
            const int e = s_ids[tid];
            int item = 0, lt = 0, cnt = 0;
            for (int q = 0; q < np; ++q) {
                const int f = s_ids[q];
                item += s_first[q] & (f < e);
                lt += f < e;
                cnt += f == e;
            }
            s_items[item] = make_int4(e, lt, cnt, 0);
        }
        if (tid == 0) {
            int n = 0;
            for (int q = 0; q < np; ++q) n += s_first[q];
            s_misc[0] = n;
        }
        if (last && blockIdx.x == 0) { // per-expert offsets for the routing sink
            int lt = 0;
            for (int q = 0; q < np; ++q) lt += s_ids[q] < tid;
            a.off[tid] = lt;
            if (tid == 0) a.off[QE_N_EXPERT] = np;
        }
        __syncthreads();
        const int nitems = s_misc[0];

        // first gate/up unit of this workgroup: issue its loads now
        const int half = (lane >> 4) & 1, rsel = lane >> 5;
        const int rd = blockIdx.x * 8 + wv * 2 + rsel; // first down row of this lane (if grid*8 >= 2048, the only one)
        uint4 pq[DEC_PF];
        uint16_t ps[DEC_PF];
#pragma unroll
        for (int k = 0; k < DEC_PF; ++k) {
            const int u = half + 2 * k;
            if (u < nitems && rd < QE_D) {
                const uint8_t *drow = arena + (size_t)s_items[u].x * QE_EXPERT_BYTES + QE_EXPERT_DOWN_OFF + (size_t)rd * QE_DN_ROW_BYTES;
                pq[k] = *(const uint4 *)(drow + l16 * 16);
                ps[k] = ((const uint16_t *)(drow + QE_FF_EXP / 2))[l16];
            }
        }
        uint4 dq0 = make_uint4(0, 0, 0, 0), dq1 = dq0;
        uint16_t dsc = 0;
        if (rd < QE_D) {
            const uint8_t *srow = sh_dn + (size_t)rd * QE_SH_DN_ROW_BYTES;
            dq0 = ((const uint4 *)(srow + l16 * 32))[0];
            dq1 = ((const uint4 *)(srow + l16 * 32))[1];
            dsc = ((const uint16_t *)(srow + QE_FF_SH))[l16];
        }
        for (int unit = blockIdx.x; unit < nitems * 32; unit += gridDim.x) {
            const int4 it = s_items[unit >> 5];
            const int r = (unit & 31) * 16 + wv * 4 + (lane >> 4);
            const uint8_t *base = arena + (size_t)it.x * QE_EXPERT_BYTES;
            const uint8_t *rg = base + (size_t)r * QE_GU_ROW_BYTES, *ru = base + (size_t)(QE_FF_EXP + r) * QE_GU_ROW_BYTES;
            uint4 qg[4], qu[4];
            float sg[4], su[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int b = l16 + 16 * j;
                qg[j] = *(const uint4 *)(rg + b * 16);
                qu[j] = *(const uint4 *)(ru + b * 16);
                sg[j] = f16_bits_to_f32(((const uint16_t *)(rg + QE_D / 2))[b]);
                su[j] = f16_bits_to_f32(((const uint16_t *)(ru + QE_D / 2))[b]);
            }
            nl4_blk dg[4], du[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) { dg[j] = nl4_decode_block(qg[j]); du[j] = nl4_decode_block(qu[j]); }
            for (int j = 0; j < it.z; ++j) {
                const int p = s_pairs[it.y + j], t = p / QE_K_USED;
                float G = 0.f, U = 0.f;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int b = l16 + 16 * q;
                    const uint4 x0 = *(const uint4 *)(s_xq + t * QE_D + b * 32), x1 = *(const uint4 *)(s_xq + t * QE_D + b * 32 + 16);
                    const float xsv = s_xs[t * 64 + b];
                    G = fmaf(sg[q] * xsv, (float)nl4_block_dot(dg[q], x0, x1), G);
                    U = fmaf(su[q] * xsv, (float)nl4_block_dot(du[q], x0, x1), U);
                }
                G = sum16(G);
                U = sum16(U);
                if (l16 == 0) ST_A((uint64_t *)EXH + (size_t)p * QE_FF_EXP + r, pack_tv(silu_mul(G, U), tagG));
            }
        }

        set_flag(FG, tagG);
        // ================= D: routed down + shared down + combine =================
        wait_flags(FG, tagG, a.err);
        for (int i = tid; i < np * 16; i += 256) {
            const int p = i >> 4, b = i & 15;
            float v[32];
            poll_tv<32>(EXH + (size_t)p * QE_FF_EXP + b * 32, 1, tagG, v, a.err);
            lane_quant_store(v, s_hq + p * QE_FF_EXP + b * 32, s_hs + i);
        }
        for (int i = tid; i < T * QE_FF_SH; i += 256) {
            const int t = i / QE_FF_SH, k = i % QE_FF_SH;
            float gu[2];
            poll_tv<2>(EXS + t * QE_SH_GU_ROWS + k, QE_FF_SH, tagR, gu, a.err);
            s_hsh[i] = silu_mul(gu[0], gu[1]);
        }
        __syncthreads();
        for (int rb = blockIdx.x * 8; rb < QE_D; rb += gridDim.x * 8) {
            const int r = rb + wv * 2 + rsel;
            const bool pf = rb == blockIdx.x * 8; // registers hold this row's weights
            float y[DEC_T];
#pragma unroll
            for (int t = 0; t < DEC_T; ++t) y[t] = 0.f;
#pragma unroll
            for (int k = 0; k < DEC_PF + 1; ++k) {
                // k < DEC_PF: prefetched item half+2k; k == DEC_PF: every remaining item
                for (int u = half + 2 * k; u < nitems; u += 2) {
                    const int4 it = s_items[u];
                    uint4 q;
                    uint16_t sraw;
                    if (k < DEC_PF && pf) {
                        q = pq[k < DEC_PF ? k : 0];
                        sraw = ps[k < DEC_PF ? k : 0];
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
                        for (int t = 0; t < DEC_T; ++t)
                            if (t == tp) y[t] += v;
                    }
                    if (k < DEC_PF) break; // one item per prefetch slot
                }
            }
#pragma unroll
            for (int t = 0; t < DEC_T; ++t) y[t] = y[t] + __shfl_xor(y[t], 16, 64);
            if (!pf) {
                const uint8_t *srow = sh_dn + (size_t)r * QE_SH_DN_ROW_BYTES;
                dq0 = ((const uint4 *)(srow + l16 * 32))[0];
                dq1 = ((const uint4 *)(srow + l16 * 32))[1];
                dsc = ((const uint16_t *)(srow + QE_FF_SH))[l16];
            }
            float w8[32];
            unpack_i8x32(dq0, dq1, w8);
            const float ssd = f16_bits_to_f32(dsc);
#pragma unroll
            for (int t = 0; t < DEC_T; ++t) {
                if (t >= T) break;
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < 32; ++i) acc = fmaf(w8[i], s_hsh[t * QE_FF_SH + l16 * 32 + i], acc);
                const float sd = sum16(acc * ssd);
                if ((lane & 31) == 0) {
                    const size_t o = (size_t)t * QE_D + r;
                    float res = 0.f;
                    if (a.residual) res = li == 0 ? a.x_in[o] : tv_val(LD_A((uint64_t *)src_x + o));
                    const float out = (res + s_shg[t] * sd) + y[t];
                    if (last) {
                        a.x_out[o] = out;
                        if (a.sd_out) a.sd_out[o] = sd;
                    } else {
                        ST_A(dst_x + o, pack_tv(out, tagD));
                    }
                }
            }
        }
        if (!last) set_flag(FD, tagD);
        __syncthreads(); // the LDS union is rewritten by the next layer's R stage
    }

    // the last workgroup out advances the epoch, so the next launch's tags are new
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0 && ADD_A(a.sync + SYNC_EXIT, 1u) == gridDim.x - 1) {
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
        // one workgroup per CU; at most 256 so that every workgroup owns router
        // rows (1281 rows / 4 waves) and down rows (2048 / 8), which the
        // dataflow ordering of buffer reuse relies on
        grid = cus < 256 ? cus : 256;
    }
    void *args[] = {(void *)&a};
    return hipLaunchCooperativeKernel((const void *)k_decode, dim3(grid), dim3(256), args, L_TOTAL, st);
}
