// IQ4_NL conversion of routed-expert weights on the GPU.
//
// The reference converts on the CPU (engine/qconv.cpp:202-227, convert_experts):
// each source row is widened to fp32 (dequant_rows, :17-43) and quantized by
// ggml's IQ4_NL quantizer (quant_row, :91-98: ggml_quantize_chunk with no
// importance matrix), and the fp16 scale and 16 code bytes of every 32-element
// block go to the row's scale and code areas.  ggml's algorithm per block
// (quantize_row_iq4_nl_impl, one 32-block per super-block, ntry = 7):
//   m = the first element of largest |x|; |m| < 1e-15 -> scale 0;
//   a candidate inverse scale s assigns q_j = nearest codebook entry of s*x_j
//   and is scored by S_xq = sum (x_j^2 q_j) x_j, S_qq = sum (x_j^2 q_j) q_j in
//   element order; s0 = 1/(m/127) gives d = S_xq/S_qq, best = d*S_xq; then
//   s = (t-127)/m, t = -7..7, replaces them when S_qq > 0 and
//   S_xq^2 > best*S_qq; the scale is stored as fp16 and the codes are the
//   nearest entries of (1/d)*x_j with the fp32 d.
//
// Here one thread quantizes one block, with the fp32 operations of that
// sequence in the same order (the library builds with -ffp-contract=off and
// correctly rounded division), so the bytes are identical to the CPU
// checker's.  The work is VALU-bound: 16 candidates x 32 elements against
// 1.6 bytes of HBM traffic per element.
//
// nearest(a): ggml bisects the codebook and keeps the lower of the two
// bracketing entries when a - lo < hi - a.  Both differences are exact
// wherever the comparison is close (every midpoint lies at |a| >= 4.5 and the
// entries are integers), so that test is a < (lo + hi)/2.  The brackets have
// integer ends and the midpoints are multiples of 1/2, so nearest(a) is
// constant on every half-unit slot [k/2, (k+1)/2): one LDS table of the slot
// values answers it.  The slot comes from 8a, whose floor rounded down to a
// multiple of 4 is the byte offset 4 floor(2a) of a 4-byte entry; 8a is exact
// (a power-of-two scaling), so it is 8 times the a that ggml rounds.
//
// In the candidate loop |a| <= |s m| <= 134.02 (|x_j| <= |m|, |s| <= 134/|m|)
// or a is NaN (a NaN or infinite input; v_cvt_flr_i32_f32 gives 0), so the
// table spans a in [-135.5, 135.5) and needs no clamp there.  The final pass
// uses s = 1/d, which has no such bound, and clamps.
#include "../../include/qe_moe.h"
#include "qe_kernels.h"

namespace {

constexpr int NL4_HALF = 271;          // slots k = -271 .. 270
constexpr int NL4_SLOTS = 2 * NL4_HALF; // 542 entries

__device__ inline int kv_at(int i) {
    const uint32_t w = i < 4 ? QE_NL4_W0 : i < 8 ? QE_NL4_W1 : i < 12 ? QE_NL4_W2 : QE_NL4_W3;
    return (int)(int8_t)(w >> (8 * (i & 3)));
}

// slot k holds a in [k/2, (k+1)/2): value and index of the nearest entry
__device__ inline void build_table(float *tab_q, int *tab_c) {
    for (int t = threadIdx.x; t < NL4_SLOTS; t += blockDim.x) {
        const int k = t - NL4_HALF;
        const int fl = k >> 1; // floor(a)
        int lo = 0;
        for (int i = 1; i < 16; ++i)
            if (kv_at(i) <= fl) lo = i;
        // a < (v_lo + v_hi)/2  <=>  k + 1/2 < v_lo + v_hi  <=>  k < v_lo + v_hi
        const int c = lo < 15 && k >= kv_at(lo) + kv_at(lo + 1) ? lo + 1 : lo;
        tab_q[t] = (float)kv_at(c);
        tab_c[t] = c;
    }
}

// byte offset of the slot of a, from a8 = 8a: 4 floor(2a) = floor(a8) & ~3
__device__ inline int slot_bytes(float a8) {
    int k;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(k) : "v"(a8));
    return k & ~3;
}

template <typename T> __device__ inline T tab_at(const T *tab0, int bytes) {
    return *(const T *)((const char *)tab0 + bytes);
}

// S_xq and S_qq of inverse scale s (given as s8 = 8 s), in element order
__device__ inline void nl4_fit(const float (&x)[32], const float (&w)[32], float s8, const float *tab0, float &sxq,
                               float &sqq) {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float q = tab_at(tab0, slot_bytes(s8 * x[j]));
        const float wq = w[j] * q;
        a = a + wq * x[j];
        b = b + wq * q;
    }
    sxq = a;
    sqq = b;
}

template <int TYPE>
__device__ inline void load_block(const uint8_t *src, uint32_t g, float (&x)[32]) {
    if constexpr (TYPE == QE_SRC_F32) {
        const float4 *p = (const float4 *)(src + (size_t)g * 128);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = p[i];
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
    } else if constexpr (TYPE == QE_SRC_F16 || TYPE == QE_SRC_BF16) {
        const uint4 *p = (const uint4 *)(src + (size_t)g * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint4 v = p[i];
            const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (TYPE == QE_SRC_F16) {
                    x[8 * i + 2 * k] = qe_f16_to_f32((uint16_t)w[k]);
                    x[8 * i + 2 * k + 1] = qe_f16_to_f32((uint16_t)(w[k] >> 16));
                } else {
                    x[8 * i + 2 * k] = __uint_as_float(w[k] << 16);
                    x[8 * i + 2 * k + 1] = __uint_as_float(w[k] & 0xffff0000u);
                }
            }
        }
    } else { // Q8_0: fp16 d, then 32 int8; blocks are 34 bytes, so 2-byte aligned
        const uint16_t *p = (const uint16_t *)(src + (size_t)g * 34);
        const float d = qe_f16_to_f32(p[0]);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const uint16_t v = p[1 + i];
            x[2 * i] = d * (float)(int8_t)(v & 0xff);
            x[2 * i + 1] = d * (float)(int8_t)(v >> 8);
        }
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_nl4_quant(QeNl4Args a) {
    __shared__ float s_q[NL4_SLOTS];
    __shared__ int s_c[NL4_SLOTS];
    build_table(s_q, s_c);
    __syncthreads();
    const uint32_t g = blockIdx.x * 256u + threadIdx.x;
    if (g >= a.nblk) return;
    float x[32], w[32];
    load_block<TYPE>(a.src, g, x);
    const float *q0 = s_q + NL4_HALF;

    float amax = 0.f, m = 0.f;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        w[j] = x[j] * x[j];
        if (fabsf(x[j]) > amax) { amax = fabsf(x[j]); m = x[j]; }
    }
    float d = 0.f;
    if (amax >= 1e-15f) {
        float sxq, sqq;
        nl4_fit(x, w, 8.f * (1.f / (m / 127.f)), q0, sxq, sqq);
        d = sxq / sqq;
        float best = d * sxq;
#pragma unroll 1
        for (int t = -7; t <= 7; ++t) {
            nl4_fit(x, w, 8.f * ((float)(t - 127) / m), q0, sxq, sqq);
            if (sqq > 0.f && sxq * sxq > best * sqq) {
                d = sxq / sqq;
                best = d * sxq;
            }
        }
    }
    const float s8 = 8.f * (d != 0.f ? 1.f / d : 0.f);
    const int *c0 = s_c + NL4_HALF;
    uint32_t c[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        const float a8 = fminf(fmaxf(s8 * x[j], -1080.f), 1079.f); // NaN -> -1080
        const uint32_t code = (uint32_t)tab_at(c0, slot_bytes(a8));
        c[(j & 15) >> 2] |= code << (8 * (j & 3) + (j >> 4) * 4);
    }
    const uint32_t row = g / a.nb, b = g - row * a.nb;
    const uint32_t grp = row / a.rows_per_group, r = row - grp * a.rows_per_group;
    uint8_t *dst = a.dst + (size_t)grp * a.group_stride + (size_t)r * a.row_stride;
    *(uint4 *)(dst + 16 * b) = make_uint4(c[0], c[1], c[2], c[3]);
    *(uint16_t *)(dst + 16 * a.nb + 2 * b) = qe_f32_to_f16(d);
}

} // namespace

hipError_t qe_launch_nl4_quant(const QeNl4Args &a, int src_type, hipStream_t st) {
    if (a.nblk == 0) return hipSuccess;
    const dim3 grid((a.nblk + 255) / 256), block(256);
    switch (src_type) {
    case QE_SRC_F32: k_nl4_quant<QE_SRC_F32><<<grid, block, 0, st>>>(a); break;
    case QE_SRC_F16: k_nl4_quant<QE_SRC_F16><<<grid, block, 0, st>>>(a); break;
    case QE_SRC_BF16: k_nl4_quant<QE_SRC_BF16><<<grid, block, 0, st>>>(a); break;
    case QE_SRC_Q8_0: k_nl4_quant<QE_SRC_Q8_0><<<grid, block, 0, st>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
