// CPU oracle for the Qwen3.6-35B-A3B MoE block -- TEST INFRASTRUCTURE ONLY.
//
// This library is the checker the HIP path is compared against, and the CPU
// baseline bench.py times.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg may load it; the product library never links or calls it.
//
// It restates the reference engine's CPU AVX2 MoE path and the GPU routing
// semantics around it (all citations are to the reference tree):
//   quant_x ............ engine/qe.cpp:687-703
//   cpu_dot_nl4(_x4) ... engine/qe.cpp:704-741, hsum256 at :681-686
//   expert SwiGLU ...... engine/qe.cpp:2066-2072 (h = g/(1+exp(-g))*u)
//   expert down ........ engine/qe.cpp:2085-2098 (ypc[p][r] = w_p * dot)
//   top-8 + weights .... engine/qe.cpp:1454-1483
//   dispatch ........... engine/qe.cpp:1965-1976 (stable counting sort)
//   combine ............ engine/qe.cpp:2033-2045
//   rmsnorm ............ engine/qe.cpp:159-168
//   Q8 block dot ....... engine/qe.cpp:91-100 (shared expert, fp32 activations)
// Two places define an order the reference leaves implementation-defined (its
// GPU sub-group reductions): the router dot product (canon_dot) and the RMSNorm
// sum of squares (canon_sumsq) use canonical orders defined below, which the
// HIP kernels reproduce exactly so that routing is bit-exact.
//
// Parity unpinned: nothing available here pins the reference's GPU kernel
// outputs (Intel sub-group reduction order, icpx contraction, the XMX
// accumulation of engine/qe.cpp:394-431), its oneMKL fp16 GEMM for the router
// and shared expert at T >= 16 (engine/qe.cpp:284-294), or the ggml IQ4_NL
// quantizer (qconv.cpp:93, off the hot path).  The checker follows the CPU
// AVX2 path instead; tests/test_oracle_pins.py pins each function below by
// closed forms, special cases, brute force and the routing-record fixture.
//
// Every function has a scalar form; quant_x and the NL4 block dot also have an
// AVX2 form written with the same intrinsic sequence semantics as the
// reference, and the tests require the two forms to agree bit for bit.
// Build: oracle/Makefile (g++ -O2 -mavx2 -mfma -mf16c -ffp-contract=off -fopenmp).
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <vector>

#include "../qe-qwen36-b50_amd/csrc/qe_format.h"
#include "../qe-qwen36-b50_amd/csrc/qe_synth.h"

#define ORC_API extern "C" __attribute__((visibility("default")))

static const int D = QE_D, NE = QE_N_EXPERT, K = QE_K_USED, FF = QE_FF_EXP;

// ---------------------------------------------------------------------------
// synthetic inputs (host side of the shared generator)
// ---------------------------------------------------------------------------
ORC_API void orc_gen_expert(uint64_t seed, int layer, int expert, uint8_t *out) {
    uint64_t *w = (uint64_t *)out;
    const int64_t n = (int64_t)(QE_EXPERT_BYTES / 8);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) w[i] = qe_synth_expert_word(seed, layer, expert, (uint64_t)i);
}
ORC_API void orc_gen_router(uint64_t seed, int layer, float *out) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < QE_ROUTER_ROWS; ++r)
        for (int c = 0; c < D; ++c) out[(size_t)r * D + c] = qe_synth_router(seed, layer, r, c);
}
ORC_API void orc_gen_q8(uint64_t seed, int layer, int which /*0 gate|up, 1 down*/, uint8_t *out) {
    const int cols = which == 0 ? D : QE_FF_SH;
    const size_t bytes = which == 0 ? QE_SH_GU_BYTES : QE_SH_DN_BYTES;
    const uint32_t tensor = which == 0 ? QE_T_SH_GU : QE_T_SH_DN;
    uint64_t *w = (uint64_t *)out;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)(bytes / 8); ++i) w[i] = qe_synth_q8_word(seed, layer, tensor, cols, (uint64_t)i);
}
ORC_API void orc_gen_x(uint64_t seed, int inst, float *out, int64_t n) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) out[i] = qe_synth_x(seed, inst, (uint64_t)i);
}
ORC_API void orc_gen_zipf_bias(uint64_t seed, int layer, double s, float *out) { qe_synth_zipf_bias(seed, layer, s, out); }
ORC_API uint16_t orc_f32_to_f16(float f) { return qe_f32_to_f16(f); }
ORC_API float orc_f16_to_f32(uint16_t h) { return qe_f16_to_f32(h); }
ORC_API double orc_normal(uint64_t key, uint64_t i) { return qe_normal(key, i); }
ORC_API double orc_log_unit(double u) { return qe_log_unit(u); }
ORC_API double orc_cos_turns(double t) { return qe_cos_turns(t); }
ORC_API uint64_t orc_stream_key(uint64_t seed, uint32_t t, uint32_t l, uint32_t s) { return qe_stream_key(seed, t, l, s); }
ORC_API uint64_t orc_draw(uint64_t key, uint64_t i) { return qe_draw(key, i); }

// ---------------------------------------------------------------------------
// quant_x: per-32 int8 activation quantisation (qe.cpp:687-703)
//   amax = max|x_i| over the block, d = amax/127 (fp32), id = d>0 ? 1/d : 0,
//   q_i = round-half-even(x_i * id) saturated to int8, scale xs[b] = d (fp32).
// ---------------------------------------------------------------------------
ORC_API void orc_quant_x(const float *x, int n, int8_t *xq, float *xs) {
    for (int b = 0; b < n / 32; ++b) {
        float amax = 0.f;
        for (int i = 0; i < 32; ++i) amax = std::max(amax, fabsf(x[b * 32 + i]));
        const float d = amax / 127.f, id = d > 0 ? 1.f / d : 0.f;
        xs[b] = d;
        for (int i = 0; i < 32; ++i) {
            const float v = nearbyintf(x[b * 32 + i] * id); /* default rounding: nearest even */
            const int q = (int)std::min(127.f, std::max(-128.f, v));
            xq[b * 32 + i] = (int8_t)q;
        }
    }
}

// The reference's vector form: maximum tree over |x|, cvtps_epi32(round), two
// saturating packs and the lane fix-up permute.
ORC_API void orc_quant_x_avx2(const float *x, int n, int8_t *xq, float *xs) {
    const __m256 sign = _mm256_set1_ps(-0.f);
    for (int b = 0; b < n / 32; ++b) {
        __m256 v[4], mx = _mm256_setzero_ps();
        for (int i = 0; i < 4; ++i) {
            v[i] = _mm256_loadu_ps(x + b * 32 + i * 8);
            mx = _mm256_max_ps(mx, _mm256_andnot_ps(sign, v[i]));
        }
        __m128 m = _mm_max_ps(_mm256_castps256_ps128(mx), _mm256_extractf128_ps(mx, 1));
        m = _mm_max_ps(m, _mm_movehl_ps(m, m));
        m = _mm_max_ss(m, _mm_movehdup_ps(m));
        const float d = _mm_cvtss_f32(m) / 127.f, id = d > 0 ? 1.f / d : 0.f;
        xs[b] = d;
        const __m256 mul = _mm256_set1_ps(id);
        __m256i q32[4];
        for (int i = 0; i < 4; ++i)
            q32[i] = _mm256_cvtps_epi32(_mm256_round_ps(_mm256_mul_ps(v[i], mul), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC));
        __m256i p = _mm256_packs_epi16(_mm256_packs_epi32(q32[0], q32[1]), _mm256_packs_epi32(q32[2], q32[3]));
        p = _mm256_permutevar8x32_epi32(p, _mm256_setr_epi32(0, 4, 1, 5, 2, 6, 3, 7));
        _mm256_storeu_si256((__m256i *)(xq + b * 32), p);
    }
}

// ---------------------------------------------------------------------------
// NL4 row . int8 activations (qe.cpp:704-720, hsum256 :681-686)
//   Per block b: exact int32 p[L] = sum_{j=4L}^{4L+3} code(j)*xq(j), L = 0..7,
//   acc[L] = fma(fp16(d_w[b]) * xs[b], float(p[L]), acc[L]) for b = 0..nb-1,
//   result = ((a0+a4)+(a2+a6)) + ((a1+a5)+(a3+a7)).
// ---------------------------------------------------------------------------
static inline int nl4_code(const uint8_t *blk, int j) {
    return QE_KVALUES_NL4[j < 16 ? (blk[j] & 15) : (blk[j - 16] >> 4)];
}
static inline float hsum8(const float *a) {
    return ((a[0] + a[4]) + (a[2] + a[6])) + ((a[1] + a[5]) + (a[3] + a[7]));
}
ORC_API float orc_dot_nl4(const uint8_t *row, int cols, const int8_t *xq, const float *xs) {
    const uint16_t *sc = (const uint16_t *)(row + cols / 2);
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < cols / 32; ++b) {
        const uint8_t *blk = row + b * 16;
        const float s = qe_f16_to_f32(sc[b]) * xs[b];
        for (int L = 0; L < 8; ++L) {
            int p = 0;
            for (int j = 4 * L; j < 4 * L + 4; ++j) p += nl4_code(blk, j) * (int)xq[b * 32 + j];
            acc[L] = fmaf(s, (float)p, acc[L]);
        }
    }
    return hsum8(acc);
}
ORC_API float orc_dot_nl4_avx2(const uint8_t *row, int cols, const int8_t *xq, const float *xs) {
    const uint16_t *sc = (const uint16_t *)(row + cols / 2);
    const __m128i tbl = _mm_loadu_si128((const __m128i *)QE_KVALUES_NL4);
    const __m128i m4 = _mm_set1_epi8(0x0f);
    const __m256i ones = _mm256_set1_epi16(1);
    __m256 acc = _mm256_setzero_ps();
    for (int b = 0; b < cols / 32; ++b) {
        const __m128i raw = _mm_loadu_si128((const __m128i *)(row + b * 16));
        const __m128i lo = _mm_shuffle_epi8(tbl, _mm_and_si128(raw, m4));
        const __m128i hi = _mm_shuffle_epi8(tbl, _mm_and_si128(_mm_srli_epi16(raw, 4), m4));
        const __m256i w = _mm256_set_m128i(hi, lo);
        const __m256i xv = _mm256_loadu_si256((const __m256i *)(xq + b * 32));
        const __m256i p = _mm256_madd_epi16(_mm256_maddubs_epi16(_mm256_sign_epi8(w, w), _mm256_sign_epi8(xv, w)), ones);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(_cvtsh_ss(sc[b]) * xs[b]), _mm256_cvtepi32_ps(p), acc);
    }
    float a[8];
    _mm256_storeu_ps(a, acc);
    return hsum8(a);
}

// The same dot for n <= 4 activation rows at once, each weight block decoded
// once for all of them (the reference's cpu_dot_nl4_x4, engine/qe.cpp:722-741,
// which its batched cold-expert path calls per group of four pairs,
// :2064-2072 and :2090-2097).  Every token keeps its own eight-lane
// accumulator and its own dw * xs[b] product, so out[t] equals
// orc_dot_nl4_avx2(row, cols, xq[t], xs[t]) bit for bit.
ORC_API void orc_dot_nl4_x4_avx2(const uint8_t *row, int cols, const int8_t *const *xq, const float *const *xs, int n,
                                 float *out) {
    const uint16_t *sc = (const uint16_t *)(row + cols / 2);
    const __m128i tbl = _mm_loadu_si128((const __m128i *)QE_KVALUES_NL4);
    const __m128i m4 = _mm_set1_epi8(0x0f);
    const __m256i ones = _mm256_set1_epi16(1);
    if (n == 1) { // one token (the reference's B = 1 decode pool calls cpu_dot_nl4 itself, :777-778)
        out[0] = orc_dot_nl4_avx2(row, cols, xq[0], xs[0]);
        return;
    }
    __m256 acc[4];
    for (int t = 0; t < 4; ++t) acc[t] = _mm256_setzero_ps();
    for (int b = 0; b < cols / 32; ++b) {
        const __m128i raw = _mm_loadu_si128((const __m128i *)(row + b * 16));
        const __m256i w = _mm256_set_m128i(_mm_shuffle_epi8(tbl, _mm_and_si128(_mm_srli_epi16(raw, 4), m4)),
                                           _mm_shuffle_epi8(tbl, _mm_and_si128(raw, m4)));
        const __m256i wabs = _mm256_sign_epi8(w, w);
        const float dw = _cvtsh_ss(sc[b]);
        for (int t = 0; t < n; ++t) {
            const __m256i xv = _mm256_loadu_si256((const __m256i *)(xq[t] + b * 32));
            const __m256i p = _mm256_madd_epi16(_mm256_maddubs_epi16(wabs, _mm256_sign_epi8(xv, w)), ones);
            acc[t] = _mm256_fmadd_ps(_mm256_set1_ps(dw * xs[t][b]), _mm256_cvtepi32_ps(p), acc[t]);
        }
    }
    for (int t = 0; t < n; ++t) {
        float a[8];
        _mm256_storeu_ps(a, acc[t]);
        out[t] = hsum8(a);
    }
}

// ---------------------------------------------------------------------------
// canonical fp32 dot of length 2048 (router rows):
//   64 chunks of 32 contiguous elements, each an fma chain from 0 in index
//   order; chunk sums combined by the pairwise tree (c, c+1), (c, c+2), ...,
//   (c, c+32) -- the value an xor-butterfly over 64 lanes with offsets
//   1, 2, 4, 8, 16, 32 leaves in every lane.
// ---------------------------------------------------------------------------
static float canon_dot(const float *a, const float *b) {
    float p[64];
    for (int c = 0; c < 64; ++c) {
        float acc = 0.f;
        for (int i = 0; i < 32; ++i) acc = fmaf(a[c * 32 + i], b[c * 32 + i], acc);
        p[c] = acc;
    }
    for (int s = 1; s < 64; s *= 2)
        for (int j = 0; j < 64; j += 2 * s) p[j] = p[j] + p[j + s];
    return p[0];
}
ORC_API float orc_canon_dot(const float *a, const float *b) { return canon_dot(a, b); }

// Canonical RMSNorm sum of squares: 256 groups of 8 contiguous elements, each
// an fma chain from 0 in index order, combined by the pairwise tree over the
// groups ((g0+g1)+(g2+g3))+... -- the order the decode kernel can assemble from
// per-workgroup partials of its 8-row output groups.
static float canon_sumsq(const float *x) {
    float p[256];
    for (int g = 0; g < 256; ++g) {
        float acc = 0.f;
        for (int i = 0; i < 8; ++i) acc = fmaf(x[g * 8 + i], x[g * 8 + i], acc);
        p[g] = acc;
    }
    for (int s = 1; s < 256; s *= 2)
        for (int j = 0; j < 256; j += 2 * s) p[j] = p[j] + p[j + s];
    return p[0];
}
ORC_API float orc_canon_sumsq(const float *x) { return canon_sumsq(x); }

// RMSNorm (qe.cpp:159-168): xn = x * (1/sqrt(ss/2048 + eps)) * w.
ORC_API void orc_rmsnorm(const float *x, const float *w, int T, float *xn) {
    for (int t = 0; t < T; ++t) {
        const float *xr = x + (size_t)t * D;
        const float ss = canon_sumsq(xr);
        const float inv = 1.0f / sqrtf(ss / (float)D + QE_RMS_EPS);
        for (int i = 0; i < D; ++i) xn[(size_t)t * D + i] = (xr[i] * inv) * (w ? w[i] : 1.0f);
    }
}

// Router (qe.cpp:144-150 semantics, canonical order): logits[t][e] =
// dot(W[e], xn_t) (+ bias[e] for e < 256); row 256 is the shared-expert gate.
ORC_API void orc_router(const float *xn, const float *W, const float *bias, int T, float *logits) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)T * QE_ROUTER_ROWS; ++i) {
        const int t = (int)(i / QE_ROUTER_ROWS), e = (int)(i % QE_ROUTER_ROWS);
        float v = canon_dot(W + (size_t)e * D, xn + (size_t)t * D);
        if (bias && e < NE) v = v + bias[e];
        logits[i] = v;
    }
}

// Top-8 (qe.cpp:1454-1483), restated with the reference's 16-lane structure:
// lane l holds v[i] = logit[i*16 + l]; each round every lane takes its first
// strict maximum, the round winner is the smallest lane holding the overall
// maximum, and its value is replaced by -1e30.  Weights are the softmax over
// the 8 selected logits relative to the first; shg = sigmoid(logit[256]).
ORC_API void orc_topk(const float *logits, int T, int32_t *ids, float *wts, float *shg) {
    for (int t = 0; t < T; ++t) {
        const float *r = logits + (size_t)t * QE_ROUTER_ROWS;
        float v[16][16];
        for (int l = 0; l < 16; ++l)
            for (int i = 0; i < 16; ++i) v[l][i] = r[i * 16 + l];
        float sel[K];
        for (int k = 0; k < K; ++k) {
            float best[16];
            int bi[16];
            for (int l = 0; l < 16; ++l) {
                best[l] = -1e30f;
                bi[l] = 0;
                for (int i = 0; i < 16; ++i)
                    if (v[l][i] > best[l]) { best[l] = v[l][i]; bi[l] = i; }
            }
            float mx = best[0];
            for (int l = 1; l < 16; ++l) mx = std::max(mx, best[l]);
            int who = 16;
            for (int l = 0; l < 16; ++l)
                if (best[l] == mx) { who = l; break; }
            v[who][bi[who]] = -1e30f;
            sel[k] = mx;
            ids[t * K + k] = bi[who] * 16 + who;
        }
        float s = 0.f;
        for (int k = 0; k < K; ++k) s += expf(sel[k] - sel[0]);
        for (int k = 0; k < K; ++k) wts[t * K + k] = expf(sel[k] - sel[0]) / s;
        shg[t] = 1.f / (1.f + expf(-r[NE]));
    }
}

// Dispatch (qe.cpp:1965-1976): cnt[e] histogram, off = exclusive scan,
// pairs[fill[id[p]]++] = p for p ascending (stable within an expert).
ORC_API void orc_dispatch(const int32_t *ids, int T, int32_t *off, int32_t *pairs) {
    std::vector<int> cnt(NE, 0);
    for (int p = 0; p < T * K; ++p) cnt[ids[p]]++;
    off[0] = 0;
    for (int e = 0; e < NE; ++e) off[e + 1] = off[e] + cnt[e];
    std::vector<int> fill(off, off + NE);
    for (int p = 0; p < T * K; ++p) pairs[fill[ids[p]]++] = p;
}

// ---------------------------------------------------------------------------
// shared expert: S(x) = D_sh . (silu(G_sh x) * (U_sh x)), Q8 rows, fp32
// activations (qe.cpp:91-100 block semantics).  The checker accumulates in
// double and rounds each dot product once.
// ---------------------------------------------------------------------------
static float q8_dot_f64(const uint8_t *row, int cols, const float *x) {
    const uint16_t *sc = (const uint16_t *)(row + cols);
    double acc = 0.0;
    for (int b = 0; b < cols / 32; ++b) {
        double s = 0.0;
        for (int i = 0; i < 32; ++i) s += (double)(int8_t)row[b * 32 + i] * (double)x[b * 32 + i];
        acc += s * (double)qe_f16_to_f32(sc[b]);
    }
    return (float)acc;
}
ORC_API void orc_shared(const float *xn, int T, const uint8_t *sh_gu, const uint8_t *sh_dn, float *sd, float *hsh) {
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) {
        float h[QE_FF_SH];
        for (int r = 0; r < QE_FF_SH; ++r) {
            const float g = q8_dot_f64(sh_gu + (size_t)r * QE_SH_GU_ROW_BYTES, D, xn + (size_t)t * D);
            const float u = q8_dot_f64(sh_gu + (size_t)(QE_FF_SH + r) * QE_SH_GU_ROW_BYTES, D, xn + (size_t)t * D);
            h[r] = g / (1.f + expf(-g)) * u;
        }
        if (hsh) memcpy(hsh + (size_t)t * QE_FF_SH, h, sizeof(h));
        for (int r = 0; r < D; ++r) sd[(size_t)t * D + r] = q8_dot_f64(sh_dn + (size_t)r * QE_SH_DN_ROW_BYTES, QE_FF_SH, h);
    }
}

// ---------------------------------------------------------------------------
// routed experts (qe.cpp:2050-2101, the batched CPU expert path):
//   xq_t = quant_x(xn_t); g = dot(G_e[r], xq_t); u = dot(U_e[r], xq_t);
//   h[p][r] = g/(1+exp(-g))*u; hq_p = quant_x(h[p]);
//   yp[p][r] = w_p * dot(D_e[r], hq_p).
// experts[e] points at expert e's blob (may be NULL for unrouted experts).
// ---------------------------------------------------------------------------
typedef float (*dot_fn)(const uint8_t *, int, const int8_t *, const float *);
typedef void (*quant_fn)(const float *, int, int8_t *, float *);

static void routed_impl(const float *xn, int T, const int32_t *ids, const float *wts, const uint8_t *const *experts,
                        float *yp, float *hout, dot_fn dot, quant_fn quant) {
    std::vector<int8_t> xq((size_t)T * D);
    std::vector<float> xs((size_t)T * (D / 32));
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) quant(xn + (size_t)t * D, D, xq.data() + (size_t)t * D, xs.data() + (size_t)t * (D / 32));
#pragma omp parallel for schedule(dynamic, 1)
    for (int p = 0; p < T * K; ++p) {
        const int t = p / K;
        const uint8_t *base = experts[ids[p]];
        float h[FF];
        int8_t hq[FF];
        float hs[FF / 32];
        for (int r = 0; r < FF; ++r) {
            const float g = dot(base + (size_t)r * QE_GU_ROW_BYTES, D, xq.data() + (size_t)t * D, xs.data() + (size_t)t * (D / 32));
            const float u = dot(base + (size_t)(FF + r) * QE_GU_ROW_BYTES, D, xq.data() + (size_t)t * D, xs.data() + (size_t)t * (D / 32));
            h[r] = g / (1.f + expf(-g)) * u;
        }
        if (hout) memcpy(hout + (size_t)p * FF, h, sizeof(h));
        quant(h, FF, hq, hs);
        const uint8_t *down = base + QE_EXPERT_DOWN_OFF;
        for (int r = 0; r < D; ++r) yp[(size_t)p * D + r] = wts[p] * dot(down + (size_t)r * QE_DN_ROW_BYTES, FF, hq, hs);
    }
}
ORC_API void orc_routed(const float *xn, int T, const int32_t *ids, const float *wts, const uint8_t *const *experts,
                        float *yp, float *hout, int use_avx2) {
    if (use_avx2) routed_impl(xn, T, ids, wts, experts, yp, hout, orc_dot_nl4_avx2, orc_quant_x_avx2);
    else routed_impl(xn, T, ids, wts, experts, yp, hout, orc_dot_nl4, orc_quant_x);
}

// Combine (qe.cpp:2036-2044): out[t] = x2[t] + shg[t]*sd[t], then += yp[t*8+k]
// for k = 0..7 in order.  x2 == NULL means a zero residual (the "normed" call).
ORC_API void orc_combine(const float *x2, const float *shg, const float *sd, const float *yp, int T, float *out) {
    for (int t = 0; t < T; ++t)
        for (int r = 0; r < D; ++r) {
            const size_t i = (size_t)t * D + r;
            float acc = (x2 ? x2[i] : 0.f) + shg[t] * sd[i];
            for (int k = 0; k < K; ++k) acc += yp[((size_t)t * K + k) * D + r];
            out[i] = acc;
        }
}

// ---------------------------------------------------------------------------
// CPU baseline: one full layer with a thread pool, the reference's batched
// cold-expert structure (qe.cpp:2050-2101): per routed expert, 32-row gate/up
// tasks and 128-row down tasks from a dynamic queue; within a row the expert's
// pairs go in groups of up to four (dispatch order), and each weight block is
// decoded once per group (orc_dot_nl4_x4_avx2, the reference's
// cpu_dot_nl4_x4).  Router, top-8, dispatch, shared expert and combine run on
// the same threads.
// ---------------------------------------------------------------------------
struct BaselineLayer {
    const float *router;    /* 257 x 2048 */
    const float *bias;      /* 256 or NULL */
    const uint8_t *sh_gu, *sh_dn;
    const uint8_t *const *experts; /* 256 blob pointers */
};

static float q8_dot_f32(const uint8_t *row, int cols, const float *x) {
    const uint16_t *sc = (const uint16_t *)(row + cols);
    float acc = 0.f;
    for (int b = 0; b < cols / 32; ++b) {
        __m256 a = _mm256_setzero_ps();
        for (int i = 0; i < 32; i += 8) {
            const __m128i q = _mm_loadl_epi64((const __m128i *)(row + b * 32 + i));
            a = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q)), _mm256_loadu_ps(x + b * 32 + i), a);
        }
        float t8[8];
        _mm256_storeu_ps(t8, a);
        acc += hsum8(t8) * _cvtsh_ss(sc[b]);
    }
    return acc;
}

ORC_API double orc_baseline_layer(const float *x2, const float *post_norm, const float *router, const float *bias,
                                  const uint8_t *sh_gu, const uint8_t *sh_dn, const uint8_t *const *experts, int T,
                                  int nthreads, float *out) {
    const auto t0 = std::chrono::steady_clock::now();
    omp_set_num_threads(nthreads);
    std::vector<float> xn((size_t)T * D), logits((size_t)T * QE_ROUTER_ROWS), wts((size_t)T * K), shg(T);
    std::vector<int32_t> ids((size_t)T * K), off(NE + 1), pairs((size_t)T * K);
    std::vector<int8_t> xq((size_t)T * D), hq((size_t)T * K * FF);
    std::vector<float> xs((size_t)T * D / 32), hs((size_t)T * K * FF / 32), h((size_t)T * K * FF), yp((size_t)T * K * D),
        sd((size_t)T * D), shh((size_t)T * QE_FF_SH);
    if (post_norm) orc_rmsnorm(x2, post_norm, T, xn.data());
    else memcpy(xn.data(), x2, xn.size() * 4);
    orc_router(xn.data(), router, bias, T, logits.data());
    orc_topk(logits.data(), T, ids.data(), wts.data(), shg.data());
    orc_dispatch(ids.data(), T, off.data(), pairs.data());
#pragma omp parallel for schedule(static)
    for (int t = 0; t < T; ++t) orc_quant_x_avx2(xn.data() + (size_t)t * D, D, xq.data() + (size_t)t * D, xs.data() + (size_t)t * (D / 32));
    // shared gate/up + activation
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)T * QE_FF_SH; ++i) {
        const int t = (int)(i / QE_FF_SH), r = (int)(i % QE_FF_SH);
        const float g = q8_dot_f32(sh_gu + (size_t)r * QE_SH_GU_ROW_BYTES, D, xn.data() + (size_t)t * D);
        const float u = q8_dot_f32(sh_gu + (size_t)(QE_FF_SH + r) * QE_SH_GU_ROW_BYTES, D, xn.data() + (size_t)t * D);
        shh[i] = g / (1.f + expf(-g)) * u;
    }
    // routed gate/up: tasks of 32 rows of one expert, tokens in groups of 4
    std::vector<int> act;
    for (int e = 0; e < NE; ++e) if (off[e + 1] > off[e]) act.push_back(e);
    const int RB = 32, RD = 128;
    const int ngu = (int)act.size() * (FF / RB);
#pragma omp parallel for schedule(dynamic, 1)
    for (int task = 0; task < ngu; ++task) {
        const int e = act[task / (FF / RB)], r0 = (task % (FF / RB)) * RB;
        const uint8_t *base = experts[e];
        for (int r = r0; r < r0 + RB; ++r)
            for (int k = off[e]; k < off[e + 1]; k += 4) {
                const int n = std::min(4, off[e + 1] - k);
                const int8_t *xqg[4];
                const float *xsg[4];
                for (int i = 0; i < n; ++i) {
                    const int t = pairs[k + i] / K;
                    xqg[i] = xq.data() + (size_t)t * D;
                    xsg[i] = xs.data() + (size_t)t * (D / 32);
                }
                float g[4], u[4];
                orc_dot_nl4_x4_avx2(base + (size_t)r * QE_GU_ROW_BYTES, D, xqg, xsg, n, g);
                orc_dot_nl4_x4_avx2(base + (size_t)(FF + r) * QE_GU_ROW_BYTES, D, xqg, xsg, n, u);
                for (int i = 0; i < n; ++i) h[(size_t)pairs[k + i] * FF + r] = g[i] / (1.f + expf(-g[i])) * u[i];
            }
    }
#pragma omp parallel for schedule(static)
    for (int p = 0; p < T * K; ++p) orc_quant_x_avx2(h.data() + (size_t)p * FF, FF, hq.data() + (size_t)p * FF, hs.data() + (size_t)p * (FF / 32));
    const int nd = (int)act.size() * (D / RD);
#pragma omp parallel for schedule(dynamic, 1)
    for (int task = 0; task < nd + D / RD; ++task) {
        if (task >= nd) { // shared down rows
            const int r0 = (task - nd) * RD;
            for (int t = 0; t < T; ++t)
                for (int r = r0; r < r0 + RD; ++r)
                    sd[(size_t)t * D + r] = q8_dot_f32(sh_dn + (size_t)r * QE_SH_DN_ROW_BYTES, QE_FF_SH, shh.data() + (size_t)t * QE_FF_SH);
            continue;
        }
        const int e = act[task / (D / RD)], r0 = (task % (D / RD)) * RD;
        const uint8_t *down = experts[e] + QE_EXPERT_DOWN_OFF;
        for (int r = r0; r < r0 + RD; ++r)
            for (int k = off[e]; k < off[e + 1]; k += 4) {
                const int n = std::min(4, off[e + 1] - k);
                const int8_t *hqg[4];
                const float *hsg[4];
                for (int i = 0; i < n; ++i) {
                    const int p = pairs[k + i];
                    hqg[i] = hq.data() + (size_t)p * FF;
                    hsg[i] = hs.data() + (size_t)p * (FF / 32);
                }
                float y[4];
                orc_dot_nl4_x4_avx2(down + (size_t)r * QE_DN_ROW_BYTES, FF, hqg, hsg, n, y);
                for (int i = 0; i < n; ++i) yp[(size_t)pairs[k + i] * D + r] = wts[pairs[k + i]] * y[i];
            }
    }
    orc_combine(post_norm ? x2 : nullptr, shg.data(), sd.data(), yp.data(), T, out);
    return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

// ---------------------------------------------------------------------------
// IQ4_NL conversion of routed-expert weights (the converter, off the inference
// path).  Follows the reference converter:
//   source block -> fp32 ..... engine/qconv.cpp:17-43 (dequant_rows: F32 as is,
//                              F16 widened, Q8_0 as fp32(d) * q; BF16 through
//                              ggml's to_float, which is the exact widening)
//   NL4 row .................. engine/qconv.cpp:91-98 (ggml's block_iq4_nl, an
//                              fp16 scale + 16 code bytes, split into the row's
//                              code area and its scale area, :48)
//   expert blob .............. engine/qconv.cpp:202-227 (expert e: its 512 gate
//                              rows, 512 up rows, 2048 down rows)
// The quantizer itself is ggml's, a dependency the reference links from a
// llama.cpp checkout (README.md:42, engine/build.sh:4) whose version it does
// not record: ggml_quantize_chunk(GGML_TYPE_IQ4_NL, ..., imatrix = NULL) runs
// ggml-quants.c's quantize_iq4_nl, i.e. quantize_row_iq4_nl_impl with one
// 32-element block per super-block, no importance weights and ntry = 7, and
// best_index_int8 for the nearest codebook entry.  Restated from that
// published algorithm:
//   * m = the first element of largest |x|; a block with |m| < 1e-15 gets
//     scale 0 (and every code the nearest entry to 0, index 8);
//   * weights w_j = x_j^2; a candidate inverse scale s assigns
//     q_j = nearest(s * x_j) and yields S_xq = sum w q x, S_qq = sum w q q,
//     summed in element order with (w*q)*x and (w*q)*q;
//   * the first candidate is s = 1 / (m / 127) and its fit d = S_xq / S_qq,
//     best = d * S_xq; then s = (t - 127) / m for t = -7..7 replaces them when
//     S_qq > 0 and S_xq^2 > best * S_qq;
//   * the fp32 scale d is stored as fp16 (round to nearest even), and the codes
//     are nearest((1/d) * x_j) with the fp32 d (0 for d = 0);
//   * code byte j = code_j | code_{j+16} << 4.
// ggml's quantizer sits in libggml-base, compiled without -march flags, so its
// fp32 arithmetic is plain SSE: no contraction, which -ffp-contract=off keeps.
// Parity with ggml's own output is unpinned (no ggml build or output vectors
// exist here); tests/test_oracle_pins.py pins the nearest-entry rule by brute
// force, the search by exact-fit blocks and by the optimality of the chosen
// candidate, and the byte layout through the NL4 dot above.
// ---------------------------------------------------------------------------
enum { ORC_SRC_F32 = 0, ORC_SRC_F16 = 1, ORC_SRC_Q8_0 = 8, ORC_SRC_BF16 = 30 }; /* ggml type ids */

static int src_block_bytes(int type) {
    return type == ORC_SRC_F32 ? 128 : type == ORC_SRC_F16 || type == ORC_SRC_BF16 ? 64 : type == ORC_SRC_Q8_0 ? 34 : 0;
}

static void src_block(const uint8_t *src, int type, int64_t blk, float *x) {
    const uint8_t *p = src + blk * src_block_bytes(type);
    for (int i = 0; i < 32; ++i) {
        uint16_t h;
        uint32_t u;
        switch (type) {
        case ORC_SRC_F32: memcpy(&x[i], p + 4 * i, 4); break;
        case ORC_SRC_F16: memcpy(&h, p + 2 * i, 2); x[i] = qe_f16_to_f32(h); break;
        case ORC_SRC_BF16: memcpy(&h, p + 2 * i, 2); u = (uint32_t)h << 16; memcpy(&x[i], &u, 4); break;
        default: memcpy(&h, p, 2); x[i] = qe_f16_to_f32(h) * (float)(int8_t)p[2 + i]; break;
        }
    }
}

ORC_API int orc_nl4_nearest(float a) {
    const int8_t *v = QE_KVALUES_NL4;
    if (a <= v[0]) return 0;
    if (a >= v[15]) return 15;
    int lo = 0, hi = 15; // v[lo] <= a < v[hi]
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (a < v[mid]) hi = mid;
        else lo = mid;
    }
    return a - v[lo] < v[hi] - a ? lo : hi;
}

static void nl4_fit(const float *x, float s, float *sxq, float *sqq) {
    float a = 0.f, b = 0.f;
    for (int j = 0; j < 32; ++j) {
        const float q = QE_KVALUES_NL4[orc_nl4_nearest(s * x[j])];
        const float wq = (x[j] * x[j]) * q;
        a = a + wq * x[j];
        b = b + wq * q;
    }
    *sxq = a;
    *sqq = b;
}

/* One 32-element block: fp16 scale and 16 code bytes; returns the fp32 scale. */
ORC_API float orc_nl4_block(const float *x, uint16_t *d16, uint8_t *codes) {
    float amax = 0.f, m = 0.f;
    for (int j = 0; j < 32; ++j)
        if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); m = x[j]; }
    float d = 0.f;
    if (amax >= 1e-15f) {
        float sxq, sqq;
        nl4_fit(x, 1.f / (m / 127.f), &sxq, &sqq);
        d = sxq / sqq;
        float best = d * sxq;
        for (int t = -7; t <= 7; ++t) {
            nl4_fit(x, (float)(t - 127) / m, &sxq, &sqq);
            if (sqq > 0.f && sxq * sxq > best * sqq) { d = sxq / sqq; best = d * sxq; }
        }
    }
    *d16 = qe_f32_to_f16(d);
    const float s = d != 0.f ? 1.f / d : 0.f;
    int c[32];
    for (int j = 0; j < 32; ++j) c[j] = orc_nl4_nearest(s * x[j]);
    for (int j = 0; j < 16; ++j) codes[j] = (uint8_t)(c[j] | c[j + 16] << 4);
    return d;
}

/* rows x cols source elements (a ggml tensor of `type`, contiguous blocks) ->
 * NL4 rows of QE_NL4_ROW_BYTES(cols) bytes. */
ORC_API int orc_nl4_quantize_rows(const void *src, int type, int64_t rows, int cols, uint8_t *dst) {
    if (!src_block_bytes(type) || cols <= 0 || cols % 32) return -1;
    const int nb = cols / 32;
    const size_t rb = QE_NL4_ROW_BYTES(cols);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        uint8_t *row = dst + r * rb;
        for (int b = 0; b < nb; ++b) {
            float x[32];
            uint16_t d16;
            src_block((const uint8_t *)src, type, r * nb + b, x);
            orc_nl4_block(x, &d16, row + b * 16);
            memcpy(row + cols / 2 + 2 * b, &d16, 2);
        }
    }
    return 0;
}

/* OpenMP threads of the calling thread's later parallel regions. */
ORC_API void orc_set_threads(int n) { omp_set_num_threads(n); }

/* Expert e's blob from the layer's ffn_{gate,up,down}_exps tensors. */
ORC_API int orc_convert_expert(const void *gate, const void *up, const void *down, int type, int e, uint8_t *blob) {
    const size_t bb = (size_t)src_block_bytes(type);
    if (!bb || e < 0 || e >= NE) return -1;
    const size_t gu_src = (size_t)e * FF * (D / 32) * bb, dn_src = (size_t)e * D * (FF / 32) * bb;
    orc_nl4_quantize_rows((const uint8_t *)gate + gu_src, type, FF, D, blob);
    orc_nl4_quantize_rows((const uint8_t *)up + gu_src, type, FF, D, blob + (size_t)FF * QE_GU_ROW_BYTES);
    orc_nl4_quantize_rows((const uint8_t *)down + dn_src, type, D, FF, blob + QE_EXPERT_DOWN_OFF);
    return 0;
}
