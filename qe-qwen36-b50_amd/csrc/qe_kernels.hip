// MoE block kernels for gfx950 (wave64).
//
// Launch plans (host side in qe_api.hip):
//  * small T (<= QE_SMALL_T tokens): the persistent kernel in qe_decode.hip;
//  * large T (prefill, Engine::moe_batched, engine/qe.cpp:1957-2047):
//      k_normq; k_router_shgu (router tiles + shared gate/up tiles), k_topk
//      (+ dispatch histogram), k_disp_scatter, the routed-expert MFMA grouped
//      GEMMs of qe_prefill.hip (shared down rides with routed down), k_combine.
// Routing (RMSNorm, router dot products, top-8) follows the checker's
// canonical fp32 order exactly; expert products use exact int8 block dots
// with fp32 block scaling, so they agree with the CPU path to fp32 rounding.
#include <mutex>

#include "qe_kernels.h"

// ===========================================================================
// large T kernels
// ===========================================================================
// wave per token: xn, xq, xs, and router row 256 (the shared-expert gate) as a
// canonical wave dot while the token's xn sits in registers (lane l holds
// elements [32l, 32l+32)), so k_topk need not read xn again.  Workgroup of
// NQ_TOK tokens (one wave each): 8 from QE_NQ8_T tokens on, 4 from 1024, 2
// below (more workgroups where there are few tokens: 512 tokens, 4 -> 2,
// 7.7 -> 6.6 us; 1 token per workgroup 7.1 us).
#define NQ_RSTR (64 * 33 + 1) /* LDS row stride (floats): the rows' same element in different banks */
#ifndef QE_NQ8_T
#define QE_NQ8_T 2048
#endif
template <int NQ_TOK>
__global__ __launch_bounds__(64 * NQ_TOK) void k_normq(const float *x, int T, const float *post_norm, float *xn, int8_t *xqp,
                                                      float *xs, _Float16 *xhl, int32_t *chunk_hist, int nch, const float *W,
                                                      float *logits) {
    constexpr int WPT = 32 / NQ_TOK; // workgroups per 32-token tile
    // the workgroup's rows move through LDS: coalesced float4 loads and stores of
    // the rows, lane c of wave w working on elements [32c, 32c+32) of row w
    // (chunks padded to 33 words: conflict-free both ways)
    __shared__ float s_r[NQ_TOK * NQ_RSTR];
    // the WPT workgroups of a 32-token tile of xhl run on one XCD (b % 8):
    // b = 8 WPT G + 8 s + x -> tokens 32 (8 G + x) + NQ_TOK s .. + NQ_TOK - 1
    const int b = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6,
              t0 = 32 * (8 * (b / (8 * WPT)) + (b & 7)) + NQ_TOK * ((b >> 3) % WPT), t = t0 + wv;
    if (b < nch) // the dispatch histogram
        for (int i = tid; i < QE_N_EXPERT; i += 64 * NQ_TOK) chunk_hist[b * QE_N_EXPERT + i] = 0;
    constexpr int F4 = QE_D / 4 / (64 * NQ_TOK); // float4s of a row per thread
#pragma unroll
    for (int r = 0; r < NQ_TOK; ++r) // row r, float4s tid + 64 NQ_TOK h
#pragma unroll
        for (int h = 0; h < F4; ++h) {
            const int f = tid + 64 * NQ_TOK * h, e = 4 * f;
            if (t0 + r < T) {
                const float4 q = ((const float4 *)(x + (size_t)(t0 + r) * QE_D))[f];
                float *sp = &s_r[r * NQ_RSTR + (e >> 5) * 33 + (e & 31)];
                sp[0] = q.x; sp[1] = q.y; sp[2] = q.z; sp[3] = q.w;
            }
        }
    __syncthreads();
    float v[32];
    if (t < T) {
#pragma unroll
        for (int i = 0; i < 32; ++i) v[i] = s_r[wv * NQ_RSTR + lane * 33 + i];
        wave_norm_chunk(v, post_norm, lane);
#pragma unroll
        for (int i = 0; i < 32; ++i) s_r[wv * NQ_RSTR + lane * 33 + i] = v[i];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NQ_TOK; ++r)
#pragma unroll
        for (int h = 0; h < F4; ++h) {
            const int f = tid + 64 * NQ_TOK * h, e = 4 * f;
            if (t0 + r < T) {
                const float *sp = &s_r[r * NQ_RSTR + (e >> 5) * 33 + (e & 31)];
                ((float4 *)(xn + (size_t)(t0 + r) * QE_D))[f] = make_float4(sp[0], sp[1], sp[2], sp[3]);
            }
        }
    {   // xn as fp16 hi/lo halves in the tile order of the shared-expert MFMA tiles
        // (qe_hl_off): thread (token i = tid % NQ_TOK, q = tid / NQ_TOK) takes groups
        // j = q + 64 k (block j / 4, 8 elements 8 (j % 4) ..); the tokens' pieces of one
        // group are consecutive 16-byte slots of a chunk, so the NQ_TOK lanes of a group
        // store one aligned run of 16 NQ_TOK bytes (a whole 128-byte line at 8 tokens)
        // instead of NQ_TOK separate pieces
        const int i = tid & (NQ_TOK - 1), q = tid / NQ_TOK;
        if (t0 + i < T) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int j = q + 64 * k, bb = j >> 2, g = j & 3;
                const float *sp = &s_r[i * NQ_RSTR + bb * 33 + 8 * g];
                uint32_t hw[4], lw[4];
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const float x0 = sp[2 * m], x1 = sp[2 * m + 1];
                    const _Float16 a0 = (_Float16)x0, a1 = (_Float16)x1;
                    hw[m] = pack_h2(a0, a1);
                    lw[m] = pack_h2((_Float16)(x0 - (float)a0), (_Float16)(x1 - (float)a1));
                }
                uint8_t *dst = (uint8_t *)xhl + qe_hl_off(QE_D, t0 + i, 32 * bb + 8 * g);
                *(uint4 *)dst = make_uint4(hw[0], hw[1], hw[2], hw[3]);
                *(uint4 *)(dst + QE_HL_LO) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
            }
        }
    }
    if (t >= T) return;
    {
        const float4 *w4 = (const float4 *)(W + (size_t)QE_N_EXPERT * QE_D + lane * 32);
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 w = w4[i];
            acc = fmaf(v[4 * i], w.x, acc);
            acc = fmaf(v[4 * i + 1], w.y, acc);
            acc = fmaf(v[4 * i + 2], w.z, acc);
            acc = fmaf(v[4 * i + 3], w.w, acc);
        }
        const float lg = wave_sum_canon(acc);
        if (lane == 0) logits[(size_t)t * QE_ROUTER_ROWS + QE_N_EXPERT] = lg;
    }
    lane_quant_store_opnd(v, xqp + (size_t)t * QE_D, lane, xs + (size_t)t * (QE_D / 32) + lane);
}

static_assert(RT_SPLIT == 8, "k_topk merges eight router partials");

// Wave per token, 4 tokens per workgroup: logits (router partials merged +
// bias; row 256 came from k_normq), then top-8 (the survivors of a group-maximum
// threshold sorted in registers), weights and the shared gate
// (engine/qe.cpp:1454-1483).  The workgroup then adds its 32 expert ids
// to the dispatch histogram of its 1024-pair chunk (zeroed by k_normq), one
// global add per distinct expert.
__global__ __launch_bounds__(256) void k_topk(const float *part, const float *bias, int T, float *logits, int32_t *ids,
                                              float *wts, float *shg, int32_t *chunk_hist) {
    __shared__ int s_h[QE_N_EXPERT];
    __shared__ uint64_t s_sk[4][64]; // each wave's survivor keys
    const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (threadIdx.x < QE_N_EXPERT) s_h[threadIdx.x] = 0;
    __syncthreads();
    if (t < T) {
    const size_t n = (size_t)T * QE_N_EXPERT;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        const float *p = part + (size_t)t * QE_N_EXPERT + e;
        float s[8];
#pragma unroll
        for (int z = 0; z < 8; ++z) s[z] = p[z * n];
        float x = ((s[0] + s[1]) + (s[2] + s[3])) + ((s[4] + s[5]) + (s[6] + s[7]));
        if (bias) x = x + bias[e];
        v[j] = x;
        logits[(size_t)t * QE_ROUTER_ROWS + e] = x;
    }
    const float lg = logits[(size_t)t * QE_ROUTER_ROWS + QE_N_EXPERT];
    const int e = wave_topk_sorted(v, lg, lane, s_sk[threadIdx.x >> 6], ids + t * QE_K_USED, wts + t * QE_K_USED, shg + t);
    if (lane < QE_K_USED) atomicAdd(&s_h[e], 1);
    }
    __syncthreads();
    static_assert(1024 % (4 * QE_K_USED) == 0, "a workgroup's pairs lie in one dispatch chunk");
    if (s_h[threadIdx.x])
        atomicAdd(&chunk_hist[(blockIdx.x * 4 * QE_K_USED / 1024) * QE_N_EXPERT + threadIdx.x], s_h[threadIdx.x]);
}

// Dispatch pass 1: per-chunk (1024 pairs) expert histogram.
__global__ __launch_bounds__(1024) void k_disp_hist(const int32_t *ids, int np, int32_t *chunk_hist) {
    __shared__ int h[QE_N_EXPERT];
    const int tid = threadIdx.x, p = blockIdx.x * 1024 + tid;
    if (tid < QE_N_EXPERT) h[tid] = 0;
    __syncthreads();
    if (p < np) atomicAdd(&h[ids[p] & (QE_N_EXPERT - 1)], 1); // ids are 0..255; others reduce modulo 256, in bounds
    __syncthreads();
    if (tid < QE_N_EXPERT) chunk_hist[blockIdx.x * QE_N_EXPERT + tid] = h[tid];
}

// Dispatch pass 2: offsets and the stable scatter (engine/qe.cpp:1968-1976).
// Inside a chunk, a pair's rank among earlier same-expert pairs is the count
// in earlier waves plus its rank in its own wave (8 ballots on the id bits).
// Block 0 also writes off[] and the work items (expert, first pair, count <= TC):
// those of more than TC / 2 pairs first, n_items[0] items in all, n_items[1] of
// them big.
__global__ __launch_bounds__(1024) void k_disp_scatter(const int32_t *ids, int np, const int32_t *chunk_hist, int nch,
                                                       int tc, int32_t *off_out, int32_t *pairs, int4 *items,
                                                       int32_t *n_items, int32_t *item_done) {
    __shared__ int s_before[QE_N_EXPERT], s_off[QE_N_EXPERT];
    __shared__ int s_w[16][QE_N_EXPERT];
    __shared__ int s_part[2][4][QE_N_EXPERT];
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    {
        // expert totals and this chunk's offset within them: four threads per
        // expert, each summing every fourth chunk (independent loads in flight;
        // one thread walking all 64 chunks of 8192 tokens took ~25 us)
        const int e = tid & (QE_N_EXPERT - 1), q = tid >> 8;
        int tot = 0, bef = 0;
#pragma unroll 4
        for (int c = q; c < nch; c += 4) {
            const int v = chunk_hist[c * QE_N_EXPERT + e];
            if (c < (int)blockIdx.x) bef += v;
            tot += v;
        }
        s_part[0][q][e] = tot;
        s_part[1][q][e] = bef;
    }
    for (int i = tid; i < 16 * QE_N_EXPERT; i += 1024) (&s_w[0][0])[i] = 0;
    __syncthreads();
    // Exclusive prefix sums over the 256 experts (threads 0..255, four waves) of the
    // pair counts and, for the work items of <= tc pairs, of each expert's big and
    // small item counts: inclusive sums within each wave by shuffles, then the
    // earlier waves' totals through LDS -- two barriers where Hillis-Steele scans over
    // LDS took sixteen each.  Items: first every item of more than tc / 2 pairs (whole
    // items and large remainders), then the small remainders, each class in expert
    // order -- the longer items start first.
    __shared__ int s_wt[4][3];
    int cnt = 0, full = 0, rem = 0, nb = 0, ns = 0, ic = 0, ib = 0, is = 0;
    if (tid < QE_N_EXPERT) {
        cnt = (s_part[0][0][tid] + s_part[0][1][tid]) + (s_part[0][2][tid] + s_part[0][3][tid]);
        s_before[tid] = (s_part[1][0][tid] + s_part[1][1][tid]) + (s_part[1][2][tid] + s_part[1][3][tid]);
        full = cnt / tc;
        rem = cnt % tc;
        nb = full + (rem > tc / 2);
        ns = rem > 0 && rem <= tc / 2;
        ic = cnt;
        ib = nb;
        is = ns;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int c2 = __shfl_up(ic, d), b2 = __shfl_up(ib, d), s2 = __shfl_up(is, d);
            if (lane >= d) {
                ic += c2;
                ib += b2;
                is += s2;
            }
        }
        if (lane == 63) {
            s_wt[wv][0] = ic;
            s_wt[wv][1] = ib;
            s_wt[wv][2] = is;
        }
    }
    __syncthreads();
    int all_c = 0, all_b = 0, all_s = 0; // totals over the experts
    if (tid < QE_N_EXPERT) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (w < wv) {
                ic += s_wt[w][0];
                ib += s_wt[w][1];
                is += s_wt[w][2];
            }
            all_c += s_wt[w][0];
            all_b += s_wt[w][1];
            all_s += s_wt[w][2];
        }
        s_off[tid] = ic - cnt;
    }
    __syncthreads();
    if (blockIdx.x == 0 && tid < QE_N_EXPERT) {
        const int off = ic - cnt, bb = ib - nb;
        off_out[tid] = off;
        if (tid == 0) off_out[QE_N_EXPERT] = all_c;
        for (int c = 0; c < full; ++c) items[bb + c] = make_int4(tid, off + c * tc, tc, 0);
        if (rem > tc / 2) items[bb + full] = make_int4(tid, off + full * tc, rem, 0);
        if (ns) items[all_b + is - 1] = make_int4(tid, off + full * tc, rem, 0);
        if (tid == QE_N_EXPERT - 1) {
            n_items[0] = all_b + all_s;
            n_items[1] = all_b;
        }
        if (item_done) // the fused gate/up + down launch counts its gate/up workgroups per item
            for (int i = tid; i < all_b + all_s; i += QE_N_EXPERT) item_done[i] = 0;
    }
    const int p = blockIdx.x * 1024 + tid;
    const bool valid = p < np;
    const int e = valid ? ids[p] & (QE_N_EXPERT - 1) : 0; // as k_disp_hist
    unsigned long long peers = __ballot(valid);
#pragma unroll
    for (int bit = 0; bit < 8; ++bit) {
        const unsigned long long b = __ballot(valid && ((e >> bit) & 1));
        peers &= ((e >> bit) & 1) ? b : ~b;
    }
    const unsigned long long lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const int rank = __popcll(peers & lt);
    if (valid && rank == 0) s_w[wv][e] = __popcll(peers);
    __syncthreads();
    if (valid) {
        int cross = 0;
        for (int w = 0; w < wv; ++w) cross += s_w[w][e];
        const int dst = s_off[e] + s_before[e] + cross + rank; // < np by construction; kept in bounds regardless
        if (dst < np) pairs[dst] = p;
    }
}


// out[t][r] = x2 + shg*sd + sum_k yp[t*8+k][r]  (engine/qe.cpp:2036-2044)
__global__ __launch_bounds__(256) void k_combine(QeCombineArgs a) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)a.T * QE_D) return;
    const int t = (int)(i / QE_D), r = (int)(i % QE_D);
    float acc = (a.x2 ? a.x2[i] : 0.f) + a.shg[t] * a.sd[i];
#pragma unroll
    for (int k = 0; k < QE_K_USED; ++k) acc += a.yp[((size_t)t * QE_K_USED + k) * QE_D + r];
    a.out[i] = acc;
}

// The same combine, then the next block's input norm on the result:
// xn[t] = RMSNorm(out[t]) * nw in the canonical order of the entry norm
// (engine/qe.cpp:1280, rmsnorm_rows of the next layer's attn_norm, or :1295
// out_norm after the last).  Workgroup per token: every thread combines 8
// elements (coalesced as in k_combine) into LDS, 32-element chunks padded to 33
// words; wave 0 forms the sum of squares in the canonical order (lane c holds
// elements [32c, 32c+32): sumsq_lane32, then the tree over the lanes), and
// every thread scales its 8 elements.
__global__ __launch_bounds__(256) void k_combine_norm(QeCombineArgs a) {
    __shared__ float s_x[64 * 33];
    __shared__ float s_inv;
    const int t = blockIdx.x, tid = threadIdx.x, e0 = tid * 8;
    const size_t o = (size_t)t * QE_D + e0;
    const float g = a.shg[t];
    float v[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const float4 s4 = *(const float4 *)(a.sd + o + 4 * h);
        const float4 x4 = a.x2 ? *(const float4 *)(a.x2 + o + 4 * h) : make_float4(0.f, 0.f, 0.f, 0.f);
        v[4 * h + 0] = x4.x + g * s4.x;
        v[4 * h + 1] = x4.y + g * s4.y;
        v[4 * h + 2] = x4.z + g * s4.z;
        v[4 * h + 3] = x4.w + g * s4.w;
    }
#pragma unroll
    for (int k = 0; k < QE_K_USED; ++k) {
        const float *y = a.yp + ((size_t)t * QE_K_USED + k) * QE_D + e0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 y4 = *(const float4 *)(y + 4 * h);
            v[4 * h + 0] += y4.x;
            v[4 * h + 1] += y4.y;
            v[4 * h + 2] += y4.z;
            v[4 * h + 3] += y4.w;
        }
    }
    float4 *out = (float4 *)(a.out + o);
    out[0] = make_float4(v[0], v[1], v[2], v[3]);
    out[1] = make_float4(v[4], v[5], v[6], v[7]);
#pragma unroll
    for (int i = 0; i < 8; ++i) s_x[(e0 >> 5) * 33 + (e0 & 31) + i] = v[i];
    __syncthreads();
    if (tid < 64) {
        float c[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) c[i] = s_x[tid * 33 + i];
        const float ss = wave_sum_canon(sumsq_lane32(c));
        if (tid == 0) s_inv = 1.0f / sqrtf(ss / (float)QE_D + QE_RMS_EPS);
    }
    __syncthreads();
    const float inv = s_inv;
    const float4 w0 = *(const float4 *)(a.nw + e0), w1 = *(const float4 *)(a.nw + e0 + 4);
    float4 *xo = (float4 *)(a.xn + o);
    xo[0] = make_float4((v[0] * inv) * w0.x, (v[1] * inv) * w0.y, (v[2] * inv) * w0.z, (v[3] * inv) * w0.w);
    xo[1] = make_float4((v[4] * inv) * w1.x, (v[5] * inv) * w1.y, (v[6] * inv) * w1.z, (v[7] * inv) * w1.w);
}

// ===========================================================================
// synthetic fills (one 8-byte word per thread, grid-stride)
// ===========================================================================
__global__ void k_synth_experts(uint8_t *arena_l, uint64_t seed, int layer) {
    const uint64_t wpe = QE_EXPERT_BYTES / 8, total = wpe * QE_N_EXPERT;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x) {
        const int e = (int)(i / wpe);
        ((uint64_t *)arena_l)[i] = qe_synth_expert_word(seed, layer, e, i % wpe);
    }
}
__global__ void k_synth_router(float *router_l, uint64_t seed, int layer) {
    const int n = QE_ROUTER_ROWS * QE_D;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        router_l[i] = qe_synth_router(seed, layer, i / QE_D, i % QE_D);
}
__global__ void k_synth_q8(uint8_t *dst, uint64_t seed, int layer, uint32_t tensor, int cols, uint64_t nwords) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nwords; i += (uint64_t)gridDim.x * blockDim.x)
        ((uint64_t *)dst)[i] = qe_synth_q8_word(seed, layer, tensor, cols, i);
}
__global__ void k_synth_x(float *out, uint64_t seed, int inst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = qe_synth_x(seed, inst, (uint64_t)i);
}
__global__ void k_fill_f32(float *p, float v, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) p[i] = v;
}

// ===========================================================================
// host launchers
// ===========================================================================
#define QE_PROF(kid) ProfScope prof_scope_##kid(S.prof, kid, st)

hipError_t qe_launch_layer(const QeLayerPtrs &L, const QeScratch &S, const float *xin, bool norm, const float *x2,
                           float *out, int T, hipStream_t st, const float *exit_norm, float *exit_xn) {
    const float *pn = norm ? L.post_norm : nullptr;
    QeCombineArgs da{T, S.yp, S.sd, S.shg, x2, out, exit_norm, exit_xn};
    {
        QE_PROF(QP_NORMQ);
        const int nch = (T * QE_K_USED + 1023) / 1024;
        if (T >= QE_NQ8_T)
            k_normq<8><<<32 * ((T + 255) / 256), 512, 0, st>>>(xin, T, pn, S.xn, S.xqp, S.xs, S.xhl, S.chunk_hist, nch,
                                                                 L.router, S.logits);
        else if (T >= 1024)
            k_normq<4><<<64 * ((T + 255) / 256), 256, 0, st>>>(xin, T, pn, S.xn, S.xqp, S.xs, S.xhl, S.chunk_hist, nch,
                                                                 L.router, S.logits);
        else
            k_normq<2><<<128 * ((T + 255) / 256), 128, 0, st>>>(xin, T, pn, S.xn, S.xqp, S.xs, S.xhl, S.chunk_hist, nch,
                                                                 L.router, S.logits);
    }
    {
        QE_PROF(QP_ROUTER);
        const hipError_t e = qe_launch_router_shgu(L, S, T, st);
        if (e != hipSuccess) return e;
    }
    {
        QE_PROF(QP_TOPK);
        k_topk<<<(T + 3) / 4, 256, 0, st>>>(S.rpart, L.bias, T, S.logits, S.ids, S.wts, S.shg, S.chunk_hist);
    }
    {
        QE_PROF(QP_DISPATCH); // the histogram came with k_topk
        const int np = T * QE_K_USED, nch = (np + 1023) / 1024;
        k_disp_scatter<<<nch, 1024, 0, st>>>(S.ids, np, S.chunk_hist, nch, QE_MFMA_MC, S.off, S.pairs, S.items,
                                              S.n_items, S.item_done);
    }
    {
        QE_PROF(QP_GU); // routed gate/up, then routed down + shared down
        const hipError_t e = qe_launch_expert_mfma(L, S, T, st);
        if (e != hipSuccess) return e;
    }
    {
        QE_PROF(QP_COMBINE);
        if (exit_norm)
            k_combine_norm<<<T, 256, 0, st>>>(da);
        else
            k_combine<<<(unsigned)(((size_t)T * QE_D + 255) / 256), 256, 0, st>>>(da);
    }
    return hipGetLastError();
}

hipError_t qe_launch_dispatch(const QeScratch &S, int T, hipStream_t st) {
    const int np = T * QE_K_USED, nch = (np + 1023) / 1024;
    k_disp_hist<<<nch, 1024, 0, st>>>(S.ids, np, S.chunk_hist);
    k_disp_scatter<<<nch, 1024, 0, st>>>(S.ids, np, S.chunk_hist, nch, QE_MFMA_MC, S.off, S.pairs, S.items,
                                          S.n_items, nullptr);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Dispatch without allocation: the scratch of the two dispatch kernels (the
// per-chunk histograms and the work items) lives in a file-scope device array
// instead of a context.  Host code never passes `scratch` itself (in host code
// the name is a stand-in, not a device address): the first call on a device
// looks the array's address up with hipGetSymbolAddress, with that device
// current, and every launch on that device takes the looked-up pointer.
// Nothing in it needs zeroing: k_disp_hist writes every histogram entry the
// scatter reads, and the scatter writes the items.  Every call on a device
// shares its array, so calls that overlap on one device race.
// ---------------------------------------------------------------------------
#define NOALLOC_NCH (QE_DISPATCH_NOALLOC_T_MAX * QE_K_USED / 1024)
#define NOALLOC_ITEMS (QE_DISPATCH_NOALLOC_T_MAX * QE_K_USED / (QE_MFMA_MC / 2 + 1) + 1 + QE_N_EXPERT)
#define NOALLOC_HIST_BYTES ((size_t)NOALLOC_NCH * QE_N_EXPERT * 4)
#define NOALLOC_BYTES (NOALLOC_HIST_BYTES + (size_t)NOALLOC_ITEMS * 16 + 256)
static_assert(NOALLOC_HIST_BYTES % 256 == 0, "items start 256-byte aligned");
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

#define NOALLOC_MAX_DEV 64
static std::mutex g_noalloc_mu;
static void *g_noalloc_ptr[NOALLOC_MAX_DEV];

// Looks up the current device's copy of `scratch` once.  qe_moe_create calls it
// for its device, so a caller holding a context can capture the no-allocation
// dispatch into a graph from its first call (the lookup may load the code
// object, which a capturing stream must not see); without a context, the first
// call on a device does the lookup and has to run before any capture.
hipError_t qe_noalloc_prepare(uint8_t **base) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= NOALLOC_MAX_DEV) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
        g_noalloc_ptr[dev] = p;
    }
    if (base) *base = (uint8_t *)g_noalloc_ptr[dev];
    return hipSuccess;
}

hipError_t qe_launch_dispatch_noalloc(const int32_t *ids, int T, int32_t *off, int32_t *pairs, hipStream_t st) {
    if (T < 1 || T > QE_DISPATCH_NOALLOC_T_MAX) return hipErrorInvalidValue;
    uint8_t *base = nullptr;
    const hipError_t e = qe_noalloc_prepare(&base);
    if (e != hipSuccess) return e;
    int32_t *chunk_hist = (int32_t *)base;
    int4 *items = (int4 *)(base + NOALLOC_HIST_BYTES);
    int32_t *n_items = (int32_t *)(base + NOALLOC_HIST_BYTES + (size_t)NOALLOC_ITEMS * 16);
    const int np = T * QE_K_USED, nch = (np + 1023) / 1024;
    k_disp_hist<<<nch, 1024, 0, st>>>(ids, np, chunk_hist);
    k_disp_scatter<<<nch, 1024, 0, st>>>(ids, np, chunk_hist, nch, QE_MFMA_MC, off, pairs, items, n_items, nullptr);
    return hipGetLastError();
}

hipError_t qe_launch_synth_layer(uint8_t *arena_l, float *router_l, uint8_t *sh_gu_l, uint8_t *sh_dn_l,
                                 float *post_norm_l, uint64_t seed, int layer, hipStream_t st) {
    k_synth_experts<<<16384, 256, 0, st>>>(arena_l, seed, layer);
    k_synth_router<<<1024, 256, 0, st>>>(router_l, seed, layer);
    k_synth_q8<<<1024, 256, 0, st>>>(sh_gu_l, seed, layer, QE_T_SH_GU, QE_D, QE_SH_GU_BYTES / 8);
    k_synth_q8<<<1024, 256, 0, st>>>(sh_dn_l, seed, layer, QE_T_SH_DN, QE_FF_SH, QE_SH_DN_BYTES / 8);
    k_fill_f32<<<8, 256, 0, st>>>(post_norm_l, 1.0f, QE_D);
    return hipGetLastError();
}

hipError_t qe_launch_synth_x(float *out, uint64_t seed, int inst, int64_t n, hipStream_t st) {
    const int64_t blocks = (n + 255) / 256;
    k_synth_x<<<(unsigned)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096), 256, 0, st>>>(out, seed, inst, n);
    return hipGetLastError();
}
